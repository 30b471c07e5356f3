// GGUF v2/v3 model files on the host: the mapped file, its metadata and
// tensor table, ggml block dequantisation, and the model shape the decode
// configuration is built from. Replaces GGUFFile
// (examples/llm/model/gguf.hpp:173-215, gguf.cpp:234-645).
//
// File layout (little-endian):
//   "GGUF" | version u32 | n_tensors u64 | n_meta u64
//   n_meta    x { key: str, kind: u32, value }        str = u64 length + bytes
//   n_tensors x { name: str, n_dims: u32, dims: u64[n_dims], type: u32, offset: u64 }
//   padding to general.alignment (default 32), then the tensor data; a
//   tensor's offset counts from the start of the data.
// dims[0] is the fastest-varying axis: a linear weight [out][in] has
// dims = {in, out}, so GGUF row j is output column j.
//
// The file is mapped read-only and never copied; every string, value and
// tensor pointer refers into the mapping and lives as long as the File.
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace xp::gguf {

// ggml tensor types (on-disk values).
enum : uint32_t {
    kF32 = 0, kF16 = 1, kQ4_0 = 2, kQ4_1 = 3, kQ5_0 = 6, kQ5_1 = 7, kQ8_0 = 8, kQ8_1 = 9,
    kQ2_K = 10, kQ3_K = 11, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kQ8_K = 15, kBF16 = 30,
};

struct BlockFormat {
    const char* name;
    uint32_t elems;      // elements per block (1 for plain types); 0 = unknown type
    uint32_t bytes;      // bytes per block
    bool dequant;        // dequantize() implements it
};
const BlockFormat& block_format(uint32_t type);

// Metadata value kinds (on-disk values).
enum : uint32_t {
    kMU8 = 0, kMI8 = 1, kMU16 = 2, kMI16 = 3, kMU32 = 4, kMI32 = 5, kMF32 = 6, kMBool = 7,
    kMStr = 8, kMArr = 9, kMU64 = 10, kMI64 = 11, kMF64 = 12,
};

struct Value {
    uint32_t kind = kMU32;
    uint32_t elem = kMU32;           // element kind of an array
    uint64_t u = 0;                  // numeric scalars are readable as any of u / i / f
    int64_t i = 0;
    double f = 0.0;
    std::string_view s;
    std::vector<std::string_view> strs;   // array of strings
    std::vector<double> nums;             // numeric array, widened
    uint64_t length() const { return kind == kMArr ? (elem == kMStr ? strs.size() : nums.size()) : 0; }
};

struct Tensor {
    std::string_view name;
    uint32_t n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint32_t type = kF32;
    uint64_t offset = 0;             // from the start of the tensor data
    const uint8_t* data = nullptr;   // into the mapping
    uint64_t nbytes = 0;
    uint64_t elements() const { return dims[0] * dims[1] * dims[2] * dims[3]; }
};

// The decode-relevant keys, read under "<general.architecture>.".
struct ModelShape {
    std::string arch, name;
    uint32_t layers = 0, heads = 0, kv_heads = 0, hidden = 0, ffn = 0, context = 0;
    uint32_t key_length = 0, value_length = 0, vocab = 0, sliding_window = 0;
    float rope_base = 10000.0f, rms_eps = 1e-6f;
    uint32_t head_dim() const { return key_length ? key_length : (heads ? hidden / heads : 0); }
};

class File {
public:
    // Maps and parses `path`; throws std::runtime_error naming the problem
    // (I/O, bad magic or version, truncation, inconsistent table).
    static std::unique_ptr<File> open(const std::string& path);
    ~File();
    File(const File&) = delete;
    File& operator=(const File&) = delete;

    const std::string& path() const { return path_; }
    uint32_t version() const { return version_; }
    uint64_t alignment() const { return alignment_; }
    uint64_t data_offset() const { return data_offset_; }
    uint64_t size() const { return size_; }
    size_t n_meta() const { return meta_.size(); }
    const std::vector<Tensor>& tensors() const { return tensors_; }
    const Tensor* tensor(std::string_view name) const;
    const Value* meta(std::string_view key) const;
    ModelShape shape() const;

private:
    File() = default;
    void parse();
    std::string path_;
    int fd_ = -1;
    const uint8_t* base_ = nullptr;
    uint64_t size_ = 0;
    uint32_t version_ = 0;
    uint64_t alignment_ = 32;
    uint64_t data_offset_ = 0;
    std::vector<std::pair<std::string_view, Value>> meta_;
    std::unordered_map<std::string_view, size_t> meta_at_;
    std::vector<Tensor> tensors_;
    std::unordered_map<std::string_view, size_t> tensor_at_;
};

// n elements of `type` at src (a whole number of blocks) into dst; false for
// a type this loader does not implement or a partial block.
bool dequantize(uint32_t type, const void* src, float* dst, size_t n);

// Rows [row0, row0 + nrows) of a 2-D tensor (row length dims[0], which must be
// a whole number of blocks) into dst[nrows][dims[0]]; throws on a bad range.
void dequantize_rows(const Tensor& t, uint64_t row0, uint64_t nrows, float* dst);

float half_to_float(uint16_t h);

}  // namespace xp::gguf

// The C ABI's handle of an open model file.
struct xp_gguf {
    std::unique_ptr<xp::gguf::File> f;
};
