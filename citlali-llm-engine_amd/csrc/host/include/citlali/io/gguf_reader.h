// citlali/io/gguf_reader.h -- GGUF (v2/v3 layout) model files.
//
// Same types, members and results as the reference's GgufFile
// (include/citlali/io/gguf_reader.h:12-91, src/io/gguf_reader.cpp:152-453):
// the header, the typed key/value metadata, the tensor directory with each
// tensor's byte size from the dtype table and its absolute offset
// align(end of directory, general.alignment) + relative offset, and the same
// typed getters with their conversions and fallbacks.  The metadata value
// types are the reference's std::variant types so code written against it
// compiles unchanged.
//
// This library's own design: the file is mapped read-only once and parsed
// from memory with every read bounds-checked; tensor bytes are served as a
// view into the mapping (tensor_data), so the weight loader copies them to
// device memory without a host-side staging copy.  read_tensor_bytes keeps
// the reference's copying form.  A GgufFile is copyable; copies share the
// mapping.  load() replaces the object only when the whole file parsed.
#pragma once

#include "citlali/compute/common/dtype.h"

#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <variant>
#include <vector>

namespace citlali::io {

// GGUF metadata value type codes (gguf_reader.h:12-26).
enum class GgufMetadataType : uint32_t {
    Uint8 = 0,
    Int8 = 1,
    Uint16 = 2,
    Int16 = 3,
    Uint32 = 4,
    Int32 = 5,
    Float32 = 6,
    Bool = 7,
    String = 8,
    Array = 9,
    Uint64 = 10,
    Int64 = 11,
    Float64 = 12,
};

using GgufScalar = std::variant<uint8_t, int8_t, uint16_t, int16_t, uint32_t, int32_t, float, bool, std::string,
                                uint64_t, int64_t, double>;
using GgufArray = std::variant<std::vector<uint8_t>, std::vector<int8_t>, std::vector<uint16_t>,
                               std::vector<int16_t>, std::vector<uint32_t>, std::vector<int32_t>,
                               std::vector<float>, std::vector<bool>, std::vector<std::string>,
                               std::vector<uint64_t>, std::vector<int64_t>, std::vector<double>>;
using GgufValue = std::variant<GgufScalar, GgufArray>;

struct GgufTensorInfo {
    std::string name;
    std::vector<uint64_t> dims;   // dims[0] = innermost (in_features for a weight)
    compute::GgufTensorType type = compute::GgufTensorType::Unknown;
    uint64_t relative_offset = 0;   // from the start of the data section
    uint64_t absolute_offset = 0;   // from the start of the file
    uint64_t nbytes = 0;

    uint64_t element_count() const;   // product of dims (1 for no dims)
};

class GgufFile {
public:
    // Parses the header, metadata and tensor directory.  Throws
    // citlali::Error for a file that cannot be opened, is not GGUF, ends
    // early, or holds an unsupported metadata type or tensor type.
    void load(const std::string& model_path);

    const std::string& path() const { return path_; }
    uint32_t version() const { return version_; }
    uint64_t alignment() const { return alignment_; }   // general.alignment, default 32
    const std::vector<GgufTensorInfo>& tensors() const { return tensors_; }
    const std::unordered_map<std::string, GgufValue>& metadata() const { return metadata_; }

    // nullptr when absent; with repeated names the last entry wins.
    const GgufTensorInfo* find_tensor(const std::string& name) const;
    bool has_key(const std::string& key) const;

    // Scalar getters: `fallback` when the key is absent or of another type.
    // get_u64 takes u64, u32 and non-negative i64/i32; get_i64 takes i64,
    // i32, u64, u32; get_f64 takes f64 and f32; get_f32 is get_f64 rounded.
    std::string get_string(const std::string& key, const std::string& fallback = "") const;
    uint64_t get_u64(const std::string& key, uint64_t fallback = 0) const;
    int64_t get_i64(const std::string& key, int64_t fallback = 0) const;
    double get_f64(const std::string& key, double fallback = 0.0) const;
    float get_f32(const std::string& key, float fallback = 0.0f) const;
    bool get_bool(const std::string& key, bool fallback = false) const;

    // Array getters: empty unless the key holds an array of exactly that type.
    std::vector<std::string> get_string_array(const std::string& key) const;
    std::vector<float> get_f32_array(const std::string& key) const;
    std::vector<uint32_t> get_u32_array(const std::string& key) const;

    // The tensor's nbytes bytes from absolute_offset; throws citlali::Error
    // when they run past the end of the file.
    std::vector<uint8_t> read_tensor_bytes(const GgufTensorInfo& tensor) const;

    // No reference counterpart: the same bytes as a view into the read-only
    // mapping, valid while this object (or a copy of it) lives.
    const uint8_t* tensor_data(const GgufTensorInfo& tensor) const;
    uint64_t data_offset() const { return data_offset_; }
    uint64_t file_size() const;

private:
    struct Mapping;
    static std::shared_ptr<const Mapping> map_file(const std::string& path);
    std::shared_ptr<const Mapping> map_;
    std::string path_;
    uint32_t version_ = 0;
    uint64_t alignment_ = 32;
    uint64_t data_offset_ = 0;
    std::vector<GgufTensorInfo> tensors_;
    std::unordered_map<std::string, GgufValue> metadata_;
    std::unordered_map<std::string, size_t> tensor_index_;
};

// A scalar as `std::ostream << value` prints it; an array as "array[N]"
// (gguf_reader.cpp:436-452).
std::string metadata_value_to_string(const GgufValue& value);

}  // namespace citlali::io
