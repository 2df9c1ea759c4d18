// gguf.hpp -- GGUF checkpoint reader: the file format ggml's gguf library
// parses for the reference's GGUFLoaderVisitor
// (src/ggml/GGUFLoaderVisitor.cpp:131-430), restated from the published GGUF
// layout (versions 2 and 3):
//
//   u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count,
//   kv_count x {string key, u32 value_type, value},
//   tensor_count x {string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type,
//                   u64 offset (relative to the data section)},
//   padding to `general.alignment` (default 32), then the data section.
//
// Strings are {u64 length, bytes}; arrays {u32 element_type, u64 count,
// elements}.  Every length, count, dimension and offset is checked against
// the file before use, so a truncated or corrupt file raises GgufError
// instead of reading out of bounds.
//
// load_gguf() places a module's parameters from such a file the way the
// reference's loader does, including its three block-aligned splits of fused
// tensors: `<p>.to_qkv_mlp_proj.weight` by rows into q, k, v, mlp_in_gate,
// mlp_in_up (:238-289), `<p>.to_out.weight` by columns into attn and mlp
// (:291-330), and the feed-forward `<p>.linear_in.{weight,bias}` by rows
// (bias: by elements) into gate and up (:332-401).
#pragma once

#include <cstdint>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "modules.hpp"

namespace dit {
namespace host {

class GgufError : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

// ggml block geometry: elements per block and bytes per block (0, 0 for a
// type this reader cannot size).
void ggml_block_layout(int32_t type, int64_t* block_elems, int64_t* block_bytes);
const char* ggml_type_label(int32_t type);

struct GgufTensor {
    std::string name;
    int32_t type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};  // ne[0] fastest (ggml order)
    uint64_t offset = 0;           // absolute file offset of the data
    uint64_t nbytes = 0;
    int64_t rows() const { return ne[1] * ne[2] * ne[3]; }
    int64_t row_bytes() const { return (int64_t)(nbytes / (uint64_t)rows()); }
    // PyTorch-order shape with ggml's trailing unit dimensions dropped, as
    // the reference derives it (GGUFLoaderVisitor.cpp:217-233).
    std::vector<int64_t> shape() const;
};

// One metadata value: scalars as int / float / bool / string; arrays keep
// their element type and count, and their elements when they are strings or
// numbers.
struct GgufValue {
    uint32_t type = 0;
    int64_t i = 0;
    uint64_t u = 0;
    double f = 0;
    std::string s;
    uint32_t array_type = 0;
    uint64_t array_count = 0;
    std::vector<std::string> array_strings;
    std::vector<double> array_numbers;
};

class GgufFile {
public:
    explicit GgufFile(const std::string& path);  // a .gguf file, or the first .gguf in a directory
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    const std::string& path() const { return path_; }
    uint32_t version() const { return version_; }
    uint64_t alignment() const { return alignment_; }
    uint64_t data_offset() const { return data_offset_; }
    uint64_t file_size() const { return size_; }
    const std::vector<GgufTensor>& tensors() const { return tensors_; }
    const std::vector<std::pair<std::string, GgufValue>>& metadata() const { return kv_; }
    const GgufTensor* find(const std::string& name) const;

    // Bytes [offset, offset + n) of the file.
    void read(uint64_t offset, void* dst, size_t n) const;
    // Rows [r0, r1) of a tensor (contiguous in the file).
    std::vector<uint8_t> read_rows(const GgufTensor& t, int64_t r0, int64_t r1) const;
    // Elements [c0, c1) of every row; both ends on block boundaries.
    std::vector<uint8_t> read_cols(const GgufTensor& t, int64_t c0, int64_t c1) const;

private:
    std::string path_;
    int fd_ = -1;
    uint64_t size_ = 0;
    uint32_t version_ = 0;
    uint64_t alignment_ = 32;
    uint64_t data_offset_ = 0;
    std::vector<GgufTensor> tensors_;
    std::map<std::string, size_t> index_;
    std::vector<std::pair<std::string, GgufValue>> kv_;
};

// Where a parameter's values live in the file: a tensor and a row range, or
// a column range of every row.
struct GgufSource {
    const GgufTensor* tensor = nullptr;
    bool by_cols = false;
    int64_t begin = 0, end = 0;  // rows (by_cols false) or elements of a row
};

// Resolves parameter `name` of `shapes` (every parameter of the module:
// name -> PyTorch shape) to its source, applying the fused-tensor splits;
// throws GgufError when the file has no such tensor or its shape differs.
GgufSource gguf_source(const GgufFile& f, const std::string& name,
                       const std::map<std::string, std::vector<int64_t>>& shapes);

struct GgufLoadStats {
    size_t parameters = 0;
    size_t file_tensors_used = 0;
    uint64_t bytes_read = 0;
    std::vector<std::string> unused;  // file tensors no parameter took
};

// Places every parameter of `m` from `f` on the device, each in a buffer from
// `alloc` that the parameter keeps (HipRuntime::bind_device).  Parameter
// types: BF16 (Linear weights; a Q8_0 source is dequantised on the device),
// DT_TYPE_Q8_0_SPLIT (a Q8_0 source is repacked, a float source quantised to
// Q8_0 first), F32 (F32/F16/BF16 sources).  Temporary device buffers come
// from the runtime's backend and are freed before returning.
GgufLoadStats load_gguf(const Module& m, const GgufFile& f, HipRuntime& rt,
                        const std::function<void*(size_t)>& alloc);

}  // namespace host
}  // namespace dit
