// gguf_reader.cpp -- GgufFile over a read-only mapping of the file.
//
// Format and results follow the reference's src/io/gguf_reader.cpp:
//   header      "GGUF", u32 version, u64 tensor count, u64 metadata count (:171-182)
//   metadata    string key, u32 type, value; arrays are u32 item type, u64
//               count, items; strings are u64 length + bytes; bool is one
//               byte, non-zero = true (:21-112, :184-188)
//   directory   string name, u32 n_dims, u64 dims[n_dims], u32 type, u64
//               offset relative to the data section (:205-229)
//   data        starts at align(end of directory, general.alignment), the
//               alignment read with get_u64 and defaulting to 32 (:197, :232-239)
// Limits kept from the reference: strings and arrays of at most 2^32 bytes /
// items (:24, :38, :87); a tensor whose type has no byte size is an error
// (:222-224).  Later duplicates of a key or tensor name replace earlier ones
// in the lookups (:187, :226).
#include "citlali/io/gguf_reader.h"

#include "citlali/common.h"

#include <cstring>
#include <sstream>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

namespace citlali::io {

struct GgufFile::Mapping {
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    ~Mapping() {
        if (base && size) munmap(const_cast<uint8_t*>(base), static_cast<size_t>(size));
    }
};

namespace {

constexpr uint64_t kMaxItems = 1ull << 32;

// Bounds-checked little-endian reader over the mapped bytes.
class Cursor {
public:
    Cursor(const uint8_t* base, uint64_t size) : base_(base), size_(size) {}
    uint64_t offset() const { return off_; }

    const uint8_t* take(uint64_t n, const char* what) {
        require(n <= size_ - off_, std::string("failed to read GGUF file: ") + what + " runs past the end at byte " +
                                       std::to_string(off_));
        const uint8_t* p = base_ + off_;
        off_ += n;
        return p;
    }
    template <typename T>
    T pod(const char* what) {
        T v;
        std::memcpy(&v, take(sizeof(T), what), sizeof(T));
        return v;
    }
    std::string string(const char* what) {
        const uint64_t n = pod<uint64_t>(what);
        require(n <= kMaxItems, "GGUF string is too large");
        const uint8_t* p = take(n, what);
        return std::string(reinterpret_cast<const char*>(p), static_cast<size_t>(n));
    }
    template <typename T>
    std::vector<T> items(uint64_t count) {
        require(count <= kMaxItems, "GGUF array is too large");
        require(count <= (size_ - off_) / sizeof(T),
                "failed to read GGUF file: array runs past the end at byte " + std::to_string(off_));
        std::vector<T> v(static_cast<size_t>(count));
        if (count) std::memcpy(v.data(), take(count * sizeof(T), "array"), static_cast<size_t>(count) * sizeof(T));
        return v;
    }

private:
    const uint8_t* base_;
    uint64_t size_;
    uint64_t off_ = 0;
};

GgufScalar read_scalar(Cursor& c, GgufMetadataType t) {
    switch (t) {
        case GgufMetadataType::Uint8: return GgufScalar(std::in_place_type<uint8_t>, c.pod<uint8_t>("value"));
        case GgufMetadataType::Int8: return GgufScalar(std::in_place_type<int8_t>, c.pod<int8_t>("value"));
        case GgufMetadataType::Uint16: return GgufScalar(std::in_place_type<uint16_t>, c.pod<uint16_t>("value"));
        case GgufMetadataType::Int16: return GgufScalar(std::in_place_type<int16_t>, c.pod<int16_t>("value"));
        case GgufMetadataType::Uint32: return GgufScalar(std::in_place_type<uint32_t>, c.pod<uint32_t>("value"));
        case GgufMetadataType::Int32: return GgufScalar(std::in_place_type<int32_t>, c.pod<int32_t>("value"));
        case GgufMetadataType::Float32: return GgufScalar(std::in_place_type<float>, c.pod<float>("value"));
        case GgufMetadataType::Bool: return GgufScalar(std::in_place_type<bool>, c.pod<uint8_t>("value") != 0);
        case GgufMetadataType::String: return GgufScalar(std::in_place_type<std::string>, c.string("value"));
        case GgufMetadataType::Uint64: return GgufScalar(std::in_place_type<uint64_t>, c.pod<uint64_t>("value"));
        case GgufMetadataType::Int64: return GgufScalar(std::in_place_type<int64_t>, c.pod<int64_t>("value"));
        case GgufMetadataType::Float64: return GgufScalar(std::in_place_type<double>, c.pod<double>("value"));
        default: throw Error("unsupported GGUF metadata scalar type " + std::to_string(static_cast<uint32_t>(t)));
    }
}

GgufArray read_array(Cursor& c, GgufMetadataType item) {
    const uint64_t n = c.pod<uint64_t>("array length");
    switch (item) {
        case GgufMetadataType::Uint8: return c.items<uint8_t>(n);
        case GgufMetadataType::Int8: return c.items<int8_t>(n);
        case GgufMetadataType::Uint16: return c.items<uint16_t>(n);
        case GgufMetadataType::Int16: return c.items<int16_t>(n);
        case GgufMetadataType::Uint32: return c.items<uint32_t>(n);
        case GgufMetadataType::Int32: return c.items<int32_t>(n);
        case GgufMetadataType::Float32: return c.items<float>(n);
        case GgufMetadataType::Uint64: return c.items<uint64_t>(n);
        case GgufMetadataType::Int64: return c.items<int64_t>(n);
        case GgufMetadataType::Float64: return c.items<double>(n);
        case GgufMetadataType::Bool: {
            const std::vector<uint8_t> raw = c.items<uint8_t>(n);
            std::vector<bool> v(raw.size());
            for (size_t i = 0; i < raw.size(); ++i) v[i] = raw[i] != 0;
            return v;
        }
        case GgufMetadataType::String: {
            require(n <= kMaxItems, "GGUF array is too large");
            std::vector<std::string> v;
            // every string takes at least its 8-byte length
            v.reserve(static_cast<size_t>(n < (1u << 20) ? n : (1u << 20)));
            for (uint64_t i = 0; i < n; ++i) v.push_back(c.string("array string"));
            return v;
        }
        default: throw Error("unsupported GGUF metadata array type " + std::to_string(static_cast<uint32_t>(item)));
    }
}

GgufValue read_value(Cursor& c) {
    const auto t = static_cast<GgufMetadataType>(c.pod<uint32_t>("value type"));
    if (t == GgufMetadataType::Array) {
        const auto item = static_cast<GgufMetadataType>(c.pod<uint32_t>("array item type"));
        return GgufValue(std::in_place_type<GgufArray>, read_array(c, item));
    }
    return GgufValue(std::in_place_type<GgufScalar>, read_scalar(c, t));
}

// The reference's rounding (gguf_reader.cpp:115-120): a power-of-two mask,
// no alignment for 0.
uint64_t align_up(uint64_t v, uint64_t a) { return a == 0 ? v : (v + a - 1) & ~(a - 1); }

template <typename T>
const T* scalar_of(const GgufValue& v) {
    const GgufScalar* s = std::get_if<GgufScalar>(&v);
    return s ? std::get_if<T>(s) : nullptr;
}

template <typename T>
std::vector<T> array_of(const GgufValue& v) {
    const GgufArray* a = std::get_if<GgufArray>(&v);
    if (!a) return {};
    const std::vector<T>* e = std::get_if<std::vector<T>>(a);
    return e ? *e : std::vector<T>{};
}

}  // namespace

std::shared_ptr<const GgufFile::Mapping> GgufFile::map_file(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    require(fd >= 0, "failed to open file: " + path);
    struct stat st {};
    if (::fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        ::close(fd);
        throw Error("failed to open file: " + path);
    }
    auto m = std::make_shared<Mapping>();
    m->size = static_cast<uint64_t>(st.st_size);
    if (m->size > 0) {
        void* p = ::mmap(nullptr, static_cast<size_t>(m->size), PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            ::close(fd);
            throw Error("failed to map file: " + path);
        }
        m->base = static_cast<const uint8_t*>(p);
    }
    ::close(fd);   // the mapping stays valid
    return m;
}

uint64_t GgufTensorInfo::element_count() const {
    uint64_t n = 1;
    for (uint64_t d : dims) n *= d;
    return n;
}

void GgufFile::load(const std::string& model_path) {
    GgufFile f;
    f.path_ = model_path;
    f.map_ = map_file(model_path);
    Cursor c(f.map_->base, f.map_->size);

    require(f.map_->size >= 4 && std::memcmp(f.map_->base, "GGUF", 4) == 0, "not a GGUF file: " + model_path);
    c.take(4, "magic");
    f.version_ = c.pod<uint32_t>("version");
    const uint64_t n_tensors = c.pod<uint64_t>("tensor count");
    const uint64_t n_kv = c.pod<uint64_t>("metadata count");

    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key = c.string("metadata key");
        f.metadata_[std::move(key)] = read_value(c);
    }
    f.alignment_ = f.get_u64("general.alignment", 32);

    // each directory entry takes at least 8 + 4 + 4 + 8 bytes
    require(n_tensors <= (f.map_->size - c.offset()) / 24,
            "failed to read GGUF file: tensor directory runs past the end");
    f.tensors_.reserve(static_cast<size_t>(n_tensors));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensorInfo t;
        t.name = c.string("tensor name");
        const uint32_t n_dims = c.pod<uint32_t>("tensor rank");
        require(n_dims <= (f.map_->size - c.offset()) / 8,
                "failed to read GGUF file: tensor dims run past the end at byte " + std::to_string(c.offset()));
        t.dims.resize(n_dims);
        for (uint32_t d = 0; d < n_dims; ++d) t.dims[d] = c.pod<uint64_t>("tensor dim");
        t.type = static_cast<compute::GgufTensorType>(c.pod<uint32_t>("tensor type"));
        t.relative_offset = c.pod<uint64_t>("tensor offset");
        t.nbytes = compute::gguf_tensor_nbytes(t.type, static_cast<size_t>(t.element_count()));
        require(t.nbytes > 0, "unsupported GGUF tensor type for tensor: " + t.name + " type=" +
                                  compute::to_string(t.type));
        f.tensor_index_[t.name] = f.tensors_.size();
        f.tensors_.push_back(std::move(t));
    }
    f.data_offset_ = align_up(c.offset(), f.alignment_);
    for (GgufTensorInfo& t : f.tensors_) t.absolute_offset = f.data_offset_ + t.relative_offset;
    *this = std::move(f);
}

const GgufTensorInfo* GgufFile::find_tensor(const std::string& name) const {
    const auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

bool GgufFile::has_key(const std::string& key) const { return metadata_.count(key) != 0; }

std::string GgufFile::get_string(const std::string& key, const std::string& fallback) const {
    const auto it = metadata_.find(key);
    if (it == metadata_.end()) return fallback;
    const std::string* s = scalar_of<std::string>(it->second);
    return s ? *s : fallback;
}

uint64_t GgufFile::get_u64(const std::string& key, uint64_t fallback) const {
    const auto it = metadata_.find(key);
    if (it == metadata_.end()) return fallback;
    const GgufValue& v = it->second;
    if (const auto* x = scalar_of<uint64_t>(v)) return *x;
    if (const auto* x = scalar_of<uint32_t>(v)) return *x;
    if (const auto* x = scalar_of<int64_t>(v)) return *x >= 0 ? static_cast<uint64_t>(*x) : fallback;
    if (const auto* x = scalar_of<int32_t>(v)) return *x >= 0 ? static_cast<uint64_t>(*x) : fallback;
    return fallback;
}

int64_t GgufFile::get_i64(const std::string& key, int64_t fallback) const {
    const auto it = metadata_.find(key);
    if (it == metadata_.end()) return fallback;
    const GgufValue& v = it->second;
    if (const auto* x = scalar_of<int64_t>(v)) return *x;
    if (const auto* x = scalar_of<int32_t>(v)) return *x;
    if (const auto* x = scalar_of<uint64_t>(v)) return static_cast<int64_t>(*x);
    if (const auto* x = scalar_of<uint32_t>(v)) return static_cast<int64_t>(*x);
    return fallback;
}

double GgufFile::get_f64(const std::string& key, double fallback) const {
    const auto it = metadata_.find(key);
    if (it == metadata_.end()) return fallback;
    if (const auto* x = scalar_of<double>(it->second)) return *x;
    if (const auto* x = scalar_of<float>(it->second)) return *x;
    return fallback;
}

float GgufFile::get_f32(const std::string& key, float fallback) const {
    return static_cast<float>(get_f64(key, fallback));
}

bool GgufFile::get_bool(const std::string& key, bool fallback) const {
    const auto it = metadata_.find(key);
    if (it == metadata_.end()) return fallback;
    const bool* b = scalar_of<bool>(it->second);
    return b ? *b : fallback;
}

std::vector<std::string> GgufFile::get_string_array(const std::string& key) const {
    const auto it = metadata_.find(key);
    return it == metadata_.end() ? std::vector<std::string>{} : array_of<std::string>(it->second);
}

std::vector<float> GgufFile::get_f32_array(const std::string& key) const {
    const auto it = metadata_.find(key);
    return it == metadata_.end() ? std::vector<float>{} : array_of<float>(it->second);
}

std::vector<uint32_t> GgufFile::get_u32_array(const std::string& key) const {
    const auto it = metadata_.find(key);
    return it == metadata_.end() ? std::vector<uint32_t>{} : array_of<uint32_t>(it->second);
}

uint64_t GgufFile::file_size() const { return map_ ? map_->size : 0; }

const uint8_t* GgufFile::tensor_data(const GgufTensorInfo& tensor) const {
    require(map_ != nullptr, "GGUF file is not loaded");
    const uint64_t size = map_->size;
    require(tensor.absolute_offset <= size && tensor.nbytes <= size - tensor.absolute_offset,
            "failed to read GGUF tensor: " + tensor.name);
    return map_->base + tensor.absolute_offset;
}

std::vector<uint8_t> GgufFile::read_tensor_bytes(const GgufTensorInfo& tensor) const {
    const uint8_t* p = tensor_data(tensor);
    return std::vector<uint8_t>(p, p + tensor.nbytes);
}

std::string metadata_value_to_string(const GgufValue& value) {
    std::ostringstream out;
    if (const GgufScalar* s = std::get_if<GgufScalar>(&value)) {
        std::visit([&](const auto& v) { out << v; }, *s);
    } else if (const GgufArray* a = std::get_if<GgufArray>(&value)) {
        std::visit([&](const auto& v) { out << "array[" << v.size() << "]"; }, *a);
    }
    return out.str();
}

}  // namespace citlali::io
