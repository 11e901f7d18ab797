// JFM v2 packages, GGUF metadata and SHA-256 for the HIP Qwen2 engine.
//
// The byte contract is the reference's (docs/jfm-v2-format.md:18-90;
// runtime/engines/native/src/format.h:6-36; loader rules
// runtime/engines/native/src/engine.c:284-757). This is an independent
// implementation: the reader validates the same topology and record rules,
// the writer emits packages the reference loader accepts.
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace jfh {

// Error carrying a jf_status-compatible code (engine.h:51-58).
enum class Status : int32_t {
    Ok = 0,
    InvalidArgument = 1,
    IoError = 2,
    FormatError = 3,
    NotFound = 4,
    OutOfMemory = 5,
    DeviceError = 6,
};

class Error : public std::runtime_error {
public:
    Error(Status code, const std::string& message) : std::runtime_error(message), code_(code) {}
    Status code() const noexcept { return code_; }

private:
    Status code_;
};

// Stable JFM tensor type ids (engine.h:13-49).
enum TensorType : uint32_t {
    kF32 = 1,
    kF16 = 2,
    kQ8_0 = 7,
    kQ2_K = 9,
    kQ4_K = 11,
    kQ6_K = 13,
};

// Canonical (elements, bytes) per storage block for every stable id 1..35.
bool type_layout(uint32_t type, uint32_t* block_elements, uint32_t* block_bytes);
const char* type_name(uint32_t type);

std::array<uint8_t, 32> sha256(const void* data, size_t size);
std::string hex(const uint8_t* data, size_t size);

// A tensor view into package (or synthetic) memory.
struct TensorView {
    std::string name;
    uint32_t type = 0;
    uint32_t rank = 0;
    uint64_t shape[4] = {1, 1, 1, 1};
    int32_t layer = -1;
    const uint8_t* data = nullptr;
    uint64_t size = 0;
};

// Selected layer range of a package (jf_stage_plan, engine.h:65-72).
struct StagePlan {
    uint32_t layer_start = 0;
    uint32_t layer_end = UINT32_MAX;
    bool verify_hashes = true;
};

struct PackageStats {
    uint32_t layer_start = 0;
    uint32_t layer_end = 0;
    uint32_t layer_count = 0;
    uint64_t selected_weight_bytes = 0;
    uint64_t total_weight_bytes = 0;
    uint64_t mapped_bytes = 0;
    uint64_t selected_tensor_count = 0;
    uint64_t total_tensor_count = 0;
};

// Read-only mmapped JFM v2 package restricted to a stage range.
class Package {
public:
    static std::unique_ptr<Package> open(const std::string& dir, const StagePlan& plan);
    ~Package();
    Package(const Package&) = delete;
    Package& operator=(const Package&) = delete;

    const PackageStats& stats() const { return stats_; }
    const std::vector<TensorView>& tensors() const { return tensors_; }  // sorted by name
    const TensorView* find(const std::string& name) const;
    const uint8_t* gguf_metadata() const { return gguf_; }
    size_t gguf_metadata_size() const { return gguf_size_; }
    const std::array<uint8_t, 32>& source_sha256() const { return source_sha256_; }

private:
    Package() = default;
    struct Mapping {
        void* address;
        size_t size;
    };
    std::vector<Mapping> mappings_;
    std::vector<TensorView> tensors_;
    const uint8_t* gguf_ = nullptr;
    size_t gguf_size_ = 0;
    std::array<uint8_t, 32> source_sha256_{};
    PackageStats stats_;
};

// Minimal GGUF v3 key/value metadata (what the qwen2 path and its tokenizer
// read; the writer emits U32, F32 and Str). Bool and I32 scalars keep their
// value in u32; string and 32-bit integer arrays are kept on request.
struct GgufValue {
    enum Kind { U32, F32, Str, Bool, I32, StrArr, I32Arr } kind = U32;
    uint32_t u32 = 0;
    float f32 = 0.0F;
    std::string str;
    std::vector<std::string> strs;
    std::vector<int32_t> ints;
};

struct GgufTensorInfo {
    std::string name;
    uint32_t type = 0;
    uint32_t rank = 0;
    uint64_t shape[4] = {1, 1, 1, 1};
    uint64_t offset = 0;
};

// Parses the KV section of a GGUF header; unknown value kinds are skipped,
// and so are arrays unless `arrays` is set.
std::map<std::string, GgufValue> parse_gguf_kv(const uint8_t* data, size_t size, bool arrays = false);

// GGML type ids (the ids GGUF tensor infos carry) <-> JFM v2 tensor type ids
// (engine.h:13-44; jf_model_compile.cpp:499-531) for the types this engine
// runs; UINT32_MAX for any other.
uint32_t jfm_type_from_ggml(uint32_t ggml_type);
uint32_t ggml_type_from_jfm(uint32_t jfm_type);

// The tensor section of a GGUF v2/v3 file: tensor infos (types as GGML ids)
// and the data section's offset (header end rounded up to general.alignment).
struct GgufLayout {
    std::vector<GgufTensorInfo> tensors;
    uint64_t data_offset = 0;
    uint32_t alignment = 32;
};
GgufLayout parse_gguf_layout(const uint8_t* data, size_t size);

// A read-only memory mapping of a whole file.
class MappedFile {
public:
    static std::shared_ptr<const MappedFile> open(const std::string& path);
    ~MappedFile();
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    const uint8_t* data() const { return data_; }
    size_t size() const { return size_; }

private:
    MappedFile() = default;
    const uint8_t* data_ = nullptr;
    size_t size_ = 0;
};

// Serializes a GGUF header: magic, version 3, KVs in order, tensor infos
// (JFM type ids written as their GGML ids), padded to the 32-byte data
// alignment (the bytes before the data section).
std::vector<uint8_t> write_gguf_header(const std::vector<std::pair<std::string, GgufValue>>& kv,
                                       const std::vector<GgufTensorInfo>& tensors);

// One tensor handed to the package writer.
struct TensorBlob {
    std::string name;
    uint32_t type = 0;
    uint32_t rank = 0;
    uint64_t shape[4] = {1, 1, 1, 1};
    const uint8_t* data = nullptr;
    uint64_t size = 0;
};

// SHA-256 and size of the source GGUF a package records in its manifest: the
// GGUF header followed by the tensor payloads at 32-byte aligned offsets, in
// the order given.
std::pair<std::array<uint8_t, 32>, uint64_t> source_digest(const std::vector<uint8_t>& gguf_header,
                                                           const std::vector<TensorBlob>& tensors);

// Writes a JFM v2 package: manifest.jfm, metadata.gguf, input/output/shared and
// one segment per layer, grouped by name (runtime/compiler/jf_model_compile.cpp:612-624).
// source: the source GGUF's SHA-256 and size for the manifest; by default
// source_digest(gguf_header, tensors).
void write_package(const std::string& dir, uint32_t layer_count, const std::vector<uint8_t>& gguf_header,
                   const std::vector<TensorBlob>& tensors,
                   const std::pair<std::array<uint8_t, 32>, uint64_t>* source = nullptr);

}  // namespace jfh
