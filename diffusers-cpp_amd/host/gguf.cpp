// gguf.cpp -- GGUF checkpoint reader and parameter placement (see gguf.hpp).
#include "gguf.hpp"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstring>
#include <dirent.h>
#include <limits>
#include <memory>

#include "runtime.hpp"

namespace dit {
namespace host {

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as little-endian u32
constexpr uint64_t kMaxDims = 4;

// GGUF metadata value types (published format).
enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

uint64_t scalar_size(uint32_t t) {
    switch (t) {
        case V_U8: case V_I8: case V_BOOL: return 1;
        case V_U16: case V_I16: return 2;
        case V_U32: case V_I32: case V_F32: return 4;
        case V_U64: case V_I64: case V_F64: return 8;
        default: return 0;
    }
}

[[noreturn]] void fail(const std::string& path, const std::string& what) {
    throw GgufError("GGUF " + path + ": " + what);
}

// Sequential reader over the header region of the file, bounds-checked
// against the file size.
class Cursor {
public:
    Cursor(int fd, uint64_t size, const std::string& path) : fd_(fd), size_(size), path_(path) {}
    uint64_t pos() const { return pos_; }
    uint64_t remaining() const { return size_ - pos_; }
    void bytes(void* dst, uint64_t n, const char* what) {
        if (n > size_ || pos_ > size_ - n) fail(path_, std::string("truncated while reading ") + what);
        fill(dst, n);
    }
    template <typename T>
    T get(const char* what) {
        T v;
        bytes(&v, sizeof(T), what);
        return v;
    }
    std::string str(const char* what) {
        const uint64_t n = get<uint64_t>(what);
        if (n > size_ - pos_) fail(path_, std::string("string length past the end of the file in ") + what);
        std::string s(n, '\0');
        bytes(s.data(), n, what);
        return s;
    }
    void skip(uint64_t n, const char* what) {
        if (n > size_ - pos_) fail(path_, std::string("truncated while skipping ") + what);
        pos_ += n;
    }

private:
    void fill(void* dst, uint64_t n) {
        // Small buffered reads: the header is parsed field by field.
        uint8_t* d = static_cast<uint8_t*>(dst);
        while (n) {
            if (buf_pos_ >= buf_.size() || buf_base_ + buf_pos_ != pos_) refill();
            const uint64_t k = std::min<uint64_t>(n, buf_.size() - buf_pos_);
            std::memcpy(d, buf_.data() + buf_pos_, k);
            d += k;
            n -= k;
            buf_pos_ += k;
            pos_ += k;
        }
    }
    void refill() {
        buf_.resize((size_t)std::min<uint64_t>(1 << 16, size_ - pos_));
        uint64_t got = 0;
        while (got < buf_.size()) {
            const ssize_t r = ::pread(fd_, buf_.data() + got, buf_.size() - got, (off_t)(pos_ + got));
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) fail(path_, "read failed");
            got += (uint64_t)r;
        }
        buf_base_ = pos_;
        buf_pos_ = 0;
    }
    int fd_;
    uint64_t size_, pos_ = 0;
    const std::string& path_;
    std::vector<uint8_t> buf_;
    uint64_t buf_base_ = 0, buf_pos_ = 0;
};

double number_of(uint32_t t, const uint8_t* p) {
    switch (t) {
        case V_U8: return *p;
        case V_I8: return (int8_t)*p;
        case V_BOOL: return *p ? 1 : 0;
        case V_U16: { uint16_t v; std::memcpy(&v, p, 2); return v; }
        case V_I16: { int16_t v; std::memcpy(&v, p, 2); return v; }
        case V_U32: { uint32_t v; std::memcpy(&v, p, 4); return v; }
        case V_I32: { int32_t v; std::memcpy(&v, p, 4); return v; }
        case V_F32: { float v; std::memcpy(&v, p, 4); return v; }
        case V_U64: { uint64_t v; std::memcpy(&v, p, 8); return (double)v; }
        case V_I64: { int64_t v; std::memcpy(&v, p, 8); return (double)v; }
        case V_F64: { double v; std::memcpy(&v, p, 8); return v; }
        default: return 0;
    }
}

GgufValue read_value(Cursor& c, uint32_t type, const std::string& path, const std::string& key) {
    GgufValue v;
    v.type = type;
    const std::string what = "metadata '" + key + "'";
    if (type == V_STRING) {
        v.s = c.str(what.c_str());
    } else if (type == V_ARRAY) {
        v.array_type = c.get<uint32_t>(what.c_str());
        v.array_count = c.get<uint64_t>(what.c_str());
        if (v.array_type == V_STRING) {
            // every string takes at least its 8-byte length
            if (v.array_count > c.remaining() / 8) fail(path, "array count exceeds the file in " + what);
            for (uint64_t i = 0; i < v.array_count; ++i) v.array_strings.push_back(c.str(what.c_str()));
        } else {
            const uint64_t es = scalar_size(v.array_type);
            if (!es) fail(path, "unsupported array element type " + std::to_string(v.array_type) + " in " + what);
            if (v.array_count > UINT64_MAX / es) fail(path, "array count overflow in " + what);
            const uint64_t n = v.array_count * es;
            if (v.array_count <= 4096) {
                std::vector<uint8_t> raw((size_t)n);
                c.bytes(raw.data(), n, what.c_str());
                for (uint64_t i = 0; i < v.array_count; ++i)
                    v.array_numbers.push_back(number_of(v.array_type, raw.data() + i * es));
            } else {
                c.skip(n, what.c_str());  // long numeric arrays (e.g. token scores): count only
            }
        }
    } else {
        const uint64_t n = scalar_size(type);
        if (!n) fail(path, "unsupported value type " + std::to_string(type) + " in " + what);
        uint8_t raw[8] = {0};
        c.bytes(raw, n, what.c_str());
        v.f = number_of(type, raw);
        if (type == V_U64) std::memcpy(&v.u, raw, 8);
        else if (type == V_I64) std::memcpy(&v.i, raw, 8);
        v.i = type == V_I64 ? v.i : (int64_t)v.f;
        v.u = type == V_U64 ? v.u : (uint64_t)(v.f < 0 ? 0 : v.f);
    }
    return v;
}

bool ends_with(const std::string& s, const std::string& suf) {
    return s.size() >= suf.size() && s.compare(s.size() - suf.size(), suf.size(), suf) == 0;
}

std::string find_gguf(const std::string& path) {
    struct stat st;
    if (::stat(path.c_str(), &st) != 0) throw GgufError("GGUF " + path + ": no such file or directory");
    if (!S_ISDIR(st.st_mode)) return path;
    // The first .gguf entry of a directory, as the reference picks it
    // (GGUFLoaderVisitor.cpp:112-129); sorted here so the choice is stable.
    std::vector<std::string> names;
    if (DIR* d = ::opendir(path.c_str())) {
        while (dirent* e = ::readdir(d))
            if (ends_with(e->d_name, ".gguf")) names.push_back(e->d_name);
        ::closedir(d);
    }
    if (names.empty()) throw GgufError("GGUF " + path + ": no .gguf file in the directory");
    std::sort(names.begin(), names.end());
    return path + "/" + names.front();
}

}  // namespace

void ggml_block_layout(int32_t type, int64_t* be, int64_t* bb) {
    // ggml_type ids and block geometry (public ggml type traits).
    switch (type) {
        case 0: *be = 1; *bb = 4; return;       // F32
        case 1: *be = 1; *bb = 2; return;       // F16
        case 2: *be = 32; *bb = 18; return;     // Q4_0
        case 3: *be = 32; *bb = 20; return;     // Q4_1
        case 6: *be = 32; *bb = 22; return;     // Q5_0
        case 7: *be = 32; *bb = 24; return;     // Q5_1
        case 8: *be = 32; *bb = 34; return;     // Q8_0
        case 9: *be = 32; *bb = 36; return;     // Q8_1
        case 10: *be = 256; *bb = 84; return;   // Q2_K
        case 11: *be = 256; *bb = 110; return;  // Q3_K
        case 12: *be = 256; *bb = 144; return;  // Q4_K
        case 13: *be = 256; *bb = 176; return;  // Q5_K
        case 14: *be = 256; *bb = 210; return;  // Q6_K
        case 15: *be = 256; *bb = 292; return;  // Q8_K
        case 24: *be = 1; *bb = 1; return;      // I8
        case 25: *be = 1; *bb = 2; return;      // I16
        case 26: *be = 1; *bb = 4; return;      // I32
        case 27: *be = 1; *bb = 8; return;      // I64
        case 28: *be = 1; *bb = 8; return;      // F64
        case 30: *be = 1; *bb = 2; return;      // BF16
        default: *be = 0; *bb = 0; return;
    }
}

const char* ggml_type_label(int32_t type) {
    switch (type) {
        case 0: return "F32"; case 1: return "F16"; case 2: return "Q4_0"; case 3: return "Q4_1";
        case 6: return "Q5_0"; case 7: return "Q5_1"; case 8: return "Q8_0"; case 9: return "Q8_1";
        case 10: return "Q2_K"; case 11: return "Q3_K"; case 12: return "Q4_K"; case 13: return "Q5_K";
        case 14: return "Q6_K"; case 15: return "Q8_K"; case 24: return "I8"; case 25: return "I16";
        case 26: return "I32"; case 27: return "I64"; case 28: return "F64"; case 30: return "BF16";
        default: return "unknown";
    }
}

std::vector<int64_t> GgufTensor::shape() const {
    int nd = 0;
    for (int i = 0; i < 4; ++i)
        if (ne[i] > 1 || (i == 0 && ne[0] == 1)) nd = i + 1;
    std::vector<int64_t> s((size_t)nd);
    for (int r = 0; r < nd; ++r) s[(size_t)r] = ne[nd - 1 - r];
    return s;
}

GgufFile::GgufFile(const std::string& path_in) : path_(find_gguf(path_in)) {
    fd_ = ::open(path_.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd_ < 0) throw GgufError("GGUF " + path_ + ": cannot open (" + std::strerror(errno) + ")");
    struct stat st;
    if (::fstat(fd_, &st) != 0) {
        ::close(fd_);
        throw GgufError("GGUF " + path_ + ": cannot stat");
    }
    size_ = (uint64_t)st.st_size;
    try {
        Cursor c(fd_, size_, path_);
        if (c.get<uint32_t>("magic") != kMagic) fail(path_, "not a GGUF file (bad magic)");
        version_ = c.get<uint32_t>("version");
        if (version_ != 2 && version_ != 3) fail(path_, "unsupported GGUF version " + std::to_string(version_));
        const uint64_t n_tensors = c.get<uint64_t>("tensor count");
        const uint64_t n_kv = c.get<uint64_t>("metadata count");
        // Each entry takes at least 8 (+4) bytes: counts beyond the file are corrupt.
        if (n_tensors > size_ / 8 || n_kv > size_ / 8) fail(path_, "tensor or metadata count exceeds the file");
        for (uint64_t i = 0; i < n_kv; ++i) {
            std::string key = c.str("metadata key");
            const uint32_t t = c.get<uint32_t>("metadata type");
            GgufValue v = read_value(c, t, path_, key);
            if (key == "general.alignment") {
                if (t != V_U32 && t != V_U64 && t != V_I32)
                    fail(path_, "general.alignment must be an integer");
                if (v.u == 0 || (v.u & (v.u - 1))) fail(path_, "general.alignment must be a power of two");
                alignment_ = v.u;
            }
            kv_.emplace_back(std::move(key), std::move(v));
        }
        tensors_.resize((size_t)n_tensors);
        for (uint64_t i = 0; i < n_tensors; ++i) {
            GgufTensor& t = tensors_[(size_t)i];
            t.name = c.str("tensor name");
            const uint32_t nd = c.get<uint32_t>("tensor dims");
            if (nd == 0 || nd > kMaxDims)
                fail(path_, "tensor '" + t.name + "' has " + std::to_string(nd) + " dimensions (1..4 supported)");
            t.n_dims = (int)nd;
            uint64_t elems = 1;
            for (uint32_t d = 0; d < nd; ++d) {
                const uint64_t n = c.get<uint64_t>("tensor dims");
                if (n == 0 || n > (uint64_t)std::numeric_limits<int64_t>::max() / elems)
                    fail(path_, "tensor '" + t.name + "' has a zero or overflowing dimension");
                t.ne[d] = (int64_t)n;
                elems *= n;
            }
            t.type = (int32_t)c.get<uint32_t>("tensor type");
            const uint64_t rel = c.get<uint64_t>("tensor offset");
            int64_t be, bb;
            ggml_block_layout(t.type, &be, &bb);
            if (!be)
                fail(path_, "tensor '" + t.name + "' has unsupported ggml type " + std::to_string(t.type));
            if (t.ne[0] % be) fail(path_, "tensor '" + t.name + "': row length is not a multiple of its block size");
            // elems < 2^63, but 2-4 bytes per element can pass 2^64: a
            // wrapped byte count would slip past the end-of-file check below.
            if (elems / (uint64_t)be > std::numeric_limits<uint64_t>::max() / (uint64_t)bb)
                fail(path_, "tensor '" + t.name + "' has more bytes than 2^64");
            t.nbytes = elems / (uint64_t)be * (uint64_t)bb;
            t.offset = rel;  // made absolute below
            if (index_.count(t.name)) fail(path_, "duplicate tensor name '" + t.name + "'");
            index_[t.name] = (size_t)i;
        }
        // The data section starts at the next multiple of the alignment.
        data_offset_ = (c.pos() + alignment_ - 1) / alignment_ * alignment_;
        for (GgufTensor& t : tensors_) {
            if (t.offset % alignment_)
                fail(path_, "tensor '" + t.name + "' data offset is not a multiple of the alignment");
            if (t.offset > size_ || data_offset_ > size_ - t.offset || t.nbytes > size_ - data_offset_ - t.offset)
                fail(path_, "tensor '" + t.name + "' data lies past the end of the file");
            t.offset += data_offset_;
        }
    } catch (...) {
        ::close(fd_);
        fd_ = -1;
        throw;
    }
}

GgufFile::~GgufFile() {
    if (fd_ >= 0) ::close(fd_);
}

const GgufTensor* GgufFile::find(const std::string& name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

void GgufFile::read(uint64_t offset, void* dst, size_t n) const {
    if (offset > size_ || n > size_ - offset) fail(path_, "read past the end of the file");
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n) {
        const ssize_t r = ::pread(fd_, d, n, (off_t)offset);
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) fail(path_, "read failed");
        d += r;
        offset += (uint64_t)r;
        n -= (size_t)r;
    }
}

std::vector<uint8_t> GgufFile::read_rows(const GgufTensor& t, int64_t r0, int64_t r1) const {
    if (r0 < 0 || r1 < r0 || r1 > t.rows()) fail(path_, "row range out of bounds for '" + t.name + "'");
    const uint64_t rb = (uint64_t)t.row_bytes();
    std::vector<uint8_t> out((size_t)((uint64_t)(r1 - r0) * rb));
    read(t.offset + (uint64_t)r0 * rb, out.data(), out.size());
    return out;
}

std::vector<uint8_t> GgufFile::read_cols(const GgufTensor& t, int64_t c0, int64_t c1) const {
    int64_t be, bb;
    ggml_block_layout(t.type, &be, &bb);
    if (c0 < 0 || c1 < c0 || c1 > t.ne[0]) fail(path_, "column range out of bounds for '" + t.name + "'");
    if (c0 % be || (c1 - c0) % be)
        fail(path_, "column range [" + std::to_string(c0) + ", " + std::to_string(c1) + ") of '" + t.name +
                        "' is not aligned to its block size (" + std::to_string(be) + ")");
    const uint64_t rb = (uint64_t)t.row_bytes(), off = (uint64_t)(c0 / be * bb),
                   n = (uint64_t)((c1 - c0) / be * bb);
    std::vector<uint8_t> out((size_t)(n * (uint64_t)t.rows()));
    for (int64_t r = 0; r < t.rows(); ++r) read(t.offset + (uint64_t)r * rb + off, out.data() + r * n, n);
    return out;
}

// ---- parameter -> file tensor ------------------------------------------------

namespace {

const std::vector<int64_t>& shape_of(const std::map<std::string, std::vector<int64_t>>& shapes,
                                     const std::string& name) {
    auto it = shapes.find(name);
    if (it == shapes.end()) throw GgufError("GGUF: the module has no parameter '" + name + "'");
    return it->second;
}

std::string shape_str(const std::vector<int64_t>& s) {
    std::string r = "[";
    for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
    return r + "]";
}

const GgufTensor& need(const GgufFile& f, const std::string& name, const std::string& for_param) {
    const GgufTensor* t = f.find(name);
    if (!t) throw GgufError("GGUF: tensor '" + name + "' (for parameter '" + for_param + "') not found");
    return *t;
}

// Splits the module path `name` = <prefix>.<mid>.<part>.<leaf>.
bool split_fused(const std::string& name, const std::string& mid, const std::vector<std::string>& parts,
                 const std::string& leaf, std::string* prefix, std::string* part) {
    for (const std::string& p : parts) {
        const std::string suf = "." + mid + "." + p + "." + leaf;
        if (ends_with(name, suf)) {
            *prefix = name.substr(0, name.size() - suf.size());
            *part = p;
            return true;
        }
    }
    return false;
}

}  // namespace

GgufSource gguf_source(const GgufFile& f, const std::string& name,
                       const std::map<std::string, std::vector<int64_t>>& shapes) {
    const std::vector<int64_t>& want = shape_of(shapes, name);
    GgufSource src;
    std::string prefix, part;
    if (const GgufTensor* t = f.find(name)) {
        if (t->shape() != want)
            throw GgufError("GGUF: tensor '" + name + "' has shape " + shape_str(t->shape()) + ", the parameter " +
                            shape_str(want));
        src.tensor = t;
        src.begin = 0;
        src.end = t->rows();
        return src;
    }
    if (split_fused(name, "to_qkv_mlp_proj", {"q", "k", "v", "mlp_in_gate", "mlp_in_up"}, "weight", &prefix,
                    &part)) {
        // Rows q | k | v | gate | up of the fused projection (GGUFLoaderVisitor.cpp:238-289).
        const std::string base = prefix + ".to_qkv_mlp_proj.";
        const int64_t inner = shape_of(shapes, base + "q.weight")[0];
        const int64_t hidden = shape_of(shapes, base + "mlp_in_gate.weight")[0];
        const int64_t dim = want[1];
        const GgufTensor& t = need(f, base + "weight", name);
        if (t.shape() != std::vector<int64_t>{3 * inner + 2 * hidden, dim})
            throw GgufError("GGUF: tensor '" + t.name + "' has shape " + shape_str(t.shape()) + ", expected " +
                            shape_str({3 * inner + 2 * hidden, dim}));
        const int64_t start = part == "q" ? 0 : part == "k" ? inner : part == "v" ? 2 * inner
                            : part == "mlp_in_gate" ? 3 * inner : 3 * inner + hidden;
        src.tensor = &t;
        src.begin = start;
        src.end = start + want[0];
        return src;
    }
    if (split_fused(name, "to_out", {"attn", "mlp"}, "weight", &prefix, &part)) {
        // Columns attn | mlp of the fused output projection (:291-330).
        const std::string base = prefix + ".to_out.";
        const int64_t inner = shape_of(shapes, base + "attn.weight")[1];
        const int64_t hidden = shape_of(shapes, base + "mlp.weight")[1];
        const GgufTensor& t = need(f, base + "weight", name);
        if (t.shape() != std::vector<int64_t>{want[0], inner + hidden})
            throw GgufError("GGUF: tensor '" + t.name + "' has shape " + shape_str(t.shape()) + ", expected " +
                            shape_str({want[0], inner + hidden}));
        src.tensor = &t;
        src.by_cols = true;
        src.begin = part == "attn" ? 0 : inner;
        src.end = src.begin + want[1];
        return src;
    }
    if (ends_with(name, ".to_out.attn.bias")) {
        // The attention output bias is the fused tensor's (:322-328).
        const std::string fused = name.substr(0, name.size() - std::string(".attn.bias").size()) + ".bias";
        const GgufTensor& t = need(f, fused, name);
        if (t.shape() != want)
            throw GgufError("GGUF: tensor '" + t.name + "' has shape " + shape_str(t.shape()) + ", the parameter " +
                            shape_str(want));
        src.tensor = &t;
        src.begin = 0;
        src.end = t.rows();
        return src;
    }
    for (const char* leaf : {"weight", "bias"}) {
        for (const char* which : {"gate", "up"}) {
            const std::string suf = std::string(".linear_in_") + which + "." + leaf;
            if (!ends_with(name, suf)) continue;
            // Rows (weight) or elements (bias) gate | up of the feed-forward's
            // fused linear_in (:332-401).
            prefix = name.substr(0, name.size() - suf.size());
            const int64_t inner = want[0];
            const GgufTensor& t = need(f, prefix + ".linear_in." + leaf, name);
            const bool is_weight = std::string(leaf) == "weight";
            const std::vector<int64_t> fused =
                is_weight ? std::vector<int64_t>{2 * inner, want[1]} : std::vector<int64_t>{2 * inner};
            if (t.shape() != fused)
                throw GgufError("GGUF: tensor '" + t.name + "' has shape " + shape_str(t.shape()) + ", expected " +
                                shape_str(fused));
            src.tensor = &t;
            src.by_cols = !is_weight;
            src.begin = std::string(which) == "gate" ? 0 : inner;
            src.end = src.begin + inner;
            return src;
        }
    }
    throw GgufError("GGUF: tensor '" + name + "' not found");
}

// ---- placement ------------------------------------------------------------------

namespace {

float half_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    uint32_t u;
    if (exp == 0x1F) {
        u = sign | 0x7F800000u | (man << 13);  // inf / NaN
    } else if (exp != 0) {
        u = sign | ((exp + 112) << 23) | (man << 13);
    } else if (man == 0) {
        u = sign;
    } else {
        // subnormal: value man * 2^-24, exactly representable in fp32
        const float v = std::ldexp((float)man, -24);
        std::memcpy(&u, &v, 4);
        u |= sign;
    }
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

std::vector<float> to_f32(const std::vector<uint8_t>& raw, int32_t type, const std::string& name) {
    std::vector<float> out;
    if (type == DT_TYPE_F32) {
        out.resize(raw.size() / 4);
        std::memcpy(out.data(), raw.data(), out.size() * 4);
    } else if (type == DT_TYPE_F16 || type == DT_TYPE_BF16) {
        out.resize(raw.size() / 2);
        for (size_t i = 0; i < out.size(); ++i) {
            uint16_t h;
            std::memcpy(&h, raw.data() + 2 * i, 2);
            if (type == DT_TYPE_F16) {
                out[i] = half_to_f32(h);
            } else {
                const uint32_t u = (uint32_t)h << 16;
                std::memcpy(&out[i], &u, 4);
            }
        }
    } else {
        throw GgufError(std::string("GGUF: tensor '") + name + "' of type " + ggml_type_label(type) +
                        " cannot feed a float parameter");
    }
    return out;
}

// A device buffer freed at scope exit.
struct TempBuffer {
    dt_backend* be;
    void* p = nullptr;
    TempBuffer(dt_backend* b, size_t n) : be(b) { check(dt_buffer_alloc(be, n ? n : 1, &p), "dt_buffer_alloc"); }
    ~TempBuffer() {
        if (p) dt_buffer_free(be, p);
    }
};

void upload(void* dst, const void* src, size_t n) {
    dt_tensor t{};
    t.type = DT_TYPE_I32;  // raw bytes; only ne/nb/data matter to the copy
    t.ne[0] = (int64_t)((n + 3) / 4);
    t.ne[1] = t.ne[2] = t.ne[3] = 1;
    t.nb[0] = 4;
    t.nb[1] = t.nb[2] = t.nb[3] = (int64_t)((n + 3) / 4 * 4);
    t.data = dst;
    check(dt_tensor_set(&t, src, 0, n, nullptr), "dt_tensor_set");
}

}  // namespace

GgufLoadStats load_gguf(const Module& m, const GgufFile& f, HipRuntime& rt,
                        const std::function<void*(size_t)>& alloc) {
    std::vector<std::pair<std::string, Tensor>> ps;
    m.named_parameters(ps);
    std::map<std::string, std::vector<int64_t>> shapes;
    for (auto& p : ps) shapes[p.first] = p.second.shape();
    dt_backend* be = rt.backend();
    if (!be) throw GgufError("GGUF: placing parameters needs a device backend");
    GgufLoadStats stats;
    std::map<std::string, int> used;
    for (auto& p : ps) {
        const std::string& name = p.first;
        const Tensor& param = p.second;
        const GgufSource src = gguf_source(f, name, shapes);
        const GgufTensor& t = *src.tensor;
        used[t.name] = 1;
        std::vector<uint8_t> raw = src.by_cols ? f.read_cols(t, src.begin, src.end) : f.read_rows(t, src.begin, src.end);
        stats.bytes_read += raw.size();
        const int64_t numel = param.numel();
        const int32_t want = param.dtype();
        void* dst = nullptr;
        if (want == DT_TYPE_F32) {
            std::vector<float> v = to_f32(raw, t.type, t.name);
            dst = alloc((size_t)numel * 4);
            upload(dst, v.data(), v.size() * 4);
        } else if (want == DT_TYPE_BF16 || want == DT_TYPE_Q8_0_SPLIT) {
            if (param.ndim() != 2) throw GgufError("GGUF: parameter '" + name + "' is not a 2-D Linear weight");
            const int64_t rows = param.shape()[0], cols = param.shape()[1];
            if (t.type == DT_TYPE_Q8_0) {
                TempBuffer blocks(be, raw.size());
                upload(blocks.p, raw.data(), raw.size());
                const int64_t rb = cols / 32 * 34;
                if (want == DT_TYPE_BF16) {
                    dst = alloc((size_t)numel * 2);
                    check(dt_dequant(blocks.p, DT_TYPE_Q8_0, rows, cols, rb, dst, cols, DT_TYPE_BF16, nullptr),
                          "dt_dequant");
                } else {
                    dst = alloc((size_t)dt_q8_0_split_bytes(rows, cols));
                    check(dt_q8_0_split(blocks.p, rows, cols, rb, dst, cols,
                                        reinterpret_cast<float*>((char*)dst + dt_q8_0_split_scale_offset(rows, cols)),
                                        rows, nullptr),
                          "dt_q8_0_split");
                }
                check(dt_backend_synchronize(be), "dt_backend_synchronize");
            } else if (t.type == DT_TYPE_Q4_K && want == DT_TYPE_BF16) {
                TempBuffer blocks(be, raw.size());
                upload(blocks.p, raw.data(), raw.size());
                dst = alloc((size_t)numel * 2);
                check(dt_dequant(blocks.p, DT_TYPE_Q4_K, rows, cols, cols / 256 * 144, dst, cols, DT_TYPE_BF16,
                                 nullptr),
                      "dt_dequant");
                check(dt_backend_synchronize(be), "dt_backend_synchronize");
            } else if (t.type == DT_TYPE_F32 || t.type == DT_TYPE_F16 || t.type == DT_TYPE_BF16) {
                if (want == DT_TYPE_BF16) {
                    std::vector<uint16_t> h((size_t)numel);
                    if (t.type == DT_TYPE_BF16) {
                        std::memcpy(h.data(), raw.data(), raw.size());
                    } else {
                        const std::vector<float> v = to_f32(raw, t.type, t.name);
                        for (size_t i = 0; i < v.size(); ++i) h[i] = f32_to_bf16_rne(v[i]);
                    }
                    dst = alloc((size_t)numel * 2);
                    upload(dst, h.data(), h.size() * 2);
                } else {
                    if (cols % 32) throw GgufError("GGUF: Q8_0 weight '" + name + "' needs rows of a multiple of 32");
                    const std::vector<float> v = to_f32(raw, t.type, t.name);
                    TempBuffer f32(be, v.size() * 4), blocks(be, (size_t)(rows * (cols / 32) * 34));
                    upload(f32.p, v.data(), v.size() * 4);
                    const int64_t rb = cols / 32 * 34;
                    check(dt_quantize_q8_0((const float*)f32.p, rows, cols, cols, blocks.p, rb, nullptr),
                          "dt_quantize_q8_0");
                    dst = alloc((size_t)dt_q8_0_split_bytes(rows, cols));
                    check(dt_q8_0_split(blocks.p, rows, cols, rb, dst, cols,
                                        reinterpret_cast<float*>((char*)dst + dt_q8_0_split_scale_offset(rows, cols)),
                                        rows, nullptr),
                          "dt_q8_0_split");
                    check(dt_backend_synchronize(be), "dt_backend_synchronize");
                }
            } else {
                throw GgufError(std::string("GGUF: tensor '") + t.name + "' of type " + ggml_type_label(t.type) +
                                " cannot feed " + (want == DT_TYPE_BF16 ? "a BF16" : "a Q8_0") + " weight");
            }
        } else {
            throw GgufError("GGUF: parameter '" + name + "' has a type the loader does not place");
        }
        rt.bind_device(*param, dst);
        ++stats.parameters;
    }
    for (const GgufTensor& t : f.tensors())
        if (!used.count(t.name)) stats.unused.push_back(t.name);
    stats.file_tensors_used = used.size();
    return stats;
}

}  // namespace host
}  // namespace dit
