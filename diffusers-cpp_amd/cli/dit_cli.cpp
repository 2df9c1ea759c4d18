// dit_cli -- command-line driver of the host modules, in the role of the
// reference's test CLIs (test/utils/TestCLI.hpp, nn-cli, flux2-cli): a test
// process writes tensors to files, runs one command, and reads the outputs.
//
//   dit_cli <Command> [--name value]...
//
// Tensor files (.dtb): int32 magic 0x31425444, int32 type (ggml id), int32
// ndim, int32 reserved, int64 shape[ndim] (PyTorch order), raw contiguous
// data.  Parameters are passed as --param-<name>, outputs as --out[-<name>].
// One JSON line with graph statistics is printed on success; errors print a
// message on stderr and exit non-zero.  Checkpoints: `--gguf PATH` loads a
// GGUF file (or a directory's first .gguf) as the reference's
// GGUFLoaderVisitor does; `GgufInfo --gguf PATH` prints a file's header,
// metadata and tensor table, and `Flux2Transformer2DModel --plan-only true
// --gguf PATH` the file tensor and range each parameter would be read from.
// `HashWeights --seed S --path P --rows R [--cols C] --out FILE` writes the
// Q8_0 blocks (or, without --cols, the RMSNorm weights) that --hash-weights S
// gives parameter P, as raw bytes (no device).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <optional>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "flux2.hpp"
#include "gguf.hpp"
#include "resnet.hpp"

using namespace dit::host;

namespace {

constexpr int32_t kMagic = 0x31425444;

struct Blob {
    int32_t type = DT_TYPE_F32;
    Tensor::Shape shape;
    std::vector<uint8_t> bytes;
};

Blob read_blob(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    int32_t hdr[4];
    f.read((char*)hdr, sizeof(hdr));
    if (!f || hdr[0] != kMagic || hdr[2] < 0 || hdr[2] > 4) throw std::runtime_error("bad tensor file " + path);
    Blob b;
    b.type = hdr[1];
    if (b.type != DT_TYPE_F32 && b.type != DT_TYPE_I32 && b.type != DT_TYPE_F16 && b.type != DT_TYPE_BF16)
        throw std::runtime_error("tensor file " + path + ": element type " + std::to_string(b.type) +
                                 " (F32, F16, BF16 or I32 expected)");
    b.shape.resize(hdr[2]);
    f.read((char*)b.shape.data(), sizeof(int64_t) * hdr[2]);
    if (!f) throw std::runtime_error("truncated tensor file " + path);
    const std::streamoff data_at = f.tellg();
    f.seekg(0, std::ios::end);
    const uint64_t avail = (uint64_t)(f.tellg() - data_at);
    f.seekg(data_at);
    // Every dimension non-negative, and the payload no larger than what the
    // file holds (which also keeps the element count far from overflow).
    const uint64_t es = (b.type == DT_TYPE_F32 || b.type == DT_TYPE_I32) ? 4 : 2;
    uint64_t n = 1;
    for (int64_t d : b.shape) {
        if (d < 0 || (d > 0 && n > avail / es / (uint64_t)d))
            throw std::runtime_error("tensor file " + path + ": its shape needs more bytes than the file holds");
        n *= (uint64_t)d;
    }
    b.bytes.resize((size_t)(n * es));
    f.read((char*)b.bytes.data(), (std::streamsize)b.bytes.size());
    if (!f) throw std::runtime_error("truncated tensor file " + path);
    return b;
}

uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

// Blob bytes as `type` (F32 -> BF16 by RNE; same type passes through).
std::vector<uint8_t> convert_blob(const Blob& b, int32_t type) {
    if (b.type == type) return b.bytes;
    if (b.type == DT_TYPE_F32 && type == DT_TYPE_BF16) {
        const size_t n = b.bytes.size() / 4;
        std::vector<uint8_t> out(n * 2);
        for (size_t i = 0; i < n; ++i) {
            float f;
            std::memcpy(&f, b.bytes.data() + 4 * i, 4);
            const uint16_t h = f32_to_bf16(f);
            std::memcpy(out.data() + 2 * i, &h, 2);
        }
        return out;
    }
    throw std::runtime_error("cannot convert tensor file type " + std::to_string(b.type) + " to " +
                             std::to_string(type));
}

void write_blob(const std::string& path, int32_t type, const Tensor::Shape& shape,
                const std::vector<uint8_t>& bytes) {
    std::ofstream f(path, std::ios::binary);
    const int32_t hdr[4] = {kMagic, type, (int32_t)shape.size(), 0};
    f.write((const char*)hdr, sizeof(hdr));
    f.write((const char*)shape.data(), sizeof(int64_t) * shape.size());
    f.write((const char*)bytes.data(), (std::streamsize)bytes.size());
    if (!f) throw std::runtime_error("cannot write " + path);
}

struct Args {
    std::string command;
    std::multimap<std::string, std::string> kv;

    bool has(const std::string& k) const { return kv.count(k) > 0; }
    std::string str(const std::string& k) const {
        auto it = kv.find(k);
        if (it == kv.end()) throw std::runtime_error("missing --" + k);
        return it->second;
    }
    std::string str(const std::string& k, const std::string& def) const { return has(k) ? str(k) : def; }
    int64_t i64(const std::string& k) const { return std::stoll(str(k)); }
    int64_t i64(const std::string& k, int64_t def) const { return has(k) ? i64(k) : def; }
    float f32(const std::string& k, float def) const { return has(k) ? std::stof(str(k)) : def; }
    bool flag(const std::string& k, bool def) const {
        if (!has(k)) return def;
        const std::string v = str(k);
        return v == "true" || v == "1";
    }
    std::vector<int64_t> list(const std::string& k) const {
        std::vector<int64_t> out;
        auto r = kv.equal_range(k);
        for (auto it = r.first; it != r.second; ++it) out.push_back(std::stoll(it->second));
        return out;
    }
};

Args parse(int argc, char** argv) {
    if (argc < 2) throw std::runtime_error("usage: dit_cli <Command> [--name value]...");
    Args a;
    a.command = argv[1];
    for (int i = 2; i < argc; ++i) {
        std::string k = argv[i];
        if (k.rfind("--", 0) != 0 || i + 1 >= argc) throw std::runtime_error("bad argument " + k);
        a.kv.emplace(k.substr(2), argv[++i]);
    }
    return a;
}

// Device buffers the CLI binds to leaves itself (resident weights and
// inputs), freed when the session ends.
struct DeviceBuffers {
    dt_backend* be = nullptr;
    std::vector<void*> ptrs;
    void* alloc(size_t bytes) {
        void* p = nullptr;
        check(dt_buffer_alloc(be, bytes ? bytes : 1, &p), "dt_buffer_alloc");
        ptrs.push_back(p);
        return p;
    }
    void release(void* p) {
        auto it = std::find(ptrs.begin(), ptrs.end(), p);
        if (it != ptrs.end()) ptrs.erase(it);
        check(dt_buffer_free(be, p), "dt_buffer_free");
    }
    ~DeviceBuffers() {
        for (void* p : ptrs) dt_buffer_free(be, p);
    }
};

size_t align256(size_t n) { return (n + 255) / 256 * 256; }

// fp32 Linear weight rows on the device -> Q8_0 blocks (dt_quantize_q8_0: the
// bytes a GGUF Q8_0 tensor holds) -> the DT_TYPE_Q8_0_SPLIT layout at dst,
// through a temporary block buffer `q8` of rows * cols / 32 * 34 bytes.
void q8_split_from_f32(const float* f32, int64_t rows, int64_t cols, void* q8, void* dst) {
    const int64_t rb = cols / 32 * 34;
    check(dt_quantize_q8_0(f32, rows, cols, cols, q8, rb, nullptr), "dt_quantize_q8_0");
    check(dt_q8_0_split(q8, rows, cols, rb, dst, cols,
                        reinterpret_cast<float*>((char*)dst + dt_q8_0_split_scale_offset(rows, cols)), rows,
                        nullptr),
          "dt_q8_0_split");
}

std::string json_str(const std::string& s) {
    std::string r = "\"";
    for (unsigned char ch : s) {
        if (ch == '"' || ch == '\\') {
            r += '\\';
            r += (char)ch;
        } else if (ch < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", ch);
            r += buf;
        } else {
            r += (char)ch;
        }
    }
    return r + "\"";
}

std::string json_num(double v) {
    if (!std::isfinite(v)) return "null";
    char buf[40];
    std::snprintf(buf, sizeof buf, "%.17g", v);
    return buf;
}

float bf16_bits_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Summary of an output tensor's bytes: element count, mean and standard
// deviation (fp64), count of NaN/Inf, and the FNV-1a hash of the bytes (equal
// hashes = bit-identical outputs across runs).
struct OutputCheck {
    int64_t n = 0, nonfinite = 0;
    double mean = 0, std = 0;
    uint64_t fnv = 0xCBF29CE484222325ull;
};

OutputCheck check_output(const std::vector<uint8_t>& bytes, int32_t type) {
    OutputCheck c;
    for (uint8_t b : bytes) c.fnv = (c.fnv ^ b) * 1099511628211ull;
    double s = 0, s2 = 0;
    const size_t es = type == DT_TYPE_F32 ? 4 : 2;
    for (size_t i = 0; i + es <= bytes.size(); i += es) {
        float f;
        if (type == DT_TYPE_F32) {
            std::memcpy(&f, bytes.data() + i, 4);
        } else {
            uint16_t h;
            std::memcpy(&h, bytes.data() + i, 2);
            f = bf16_bits_to_f32(h);
        }
        ++c.n;
        if (!std::isfinite(f)) {
            ++c.nonfinite;
            continue;
        }
        s += f;
        s2 += (double)f * f;
    }
    const int64_t m = c.n - c.nonfinite;
    if (m > 0) {
        c.mean = s / m;
        c.std = std::sqrt(std::max(0.0, s2 / m - c.mean * c.mean));
    }
    return c;
}

std::string output_json(const OutputCheck& c) {
    char buf[64];
    std::snprintf(buf, sizeof buf, "\"%016llx\"", (unsigned long long)c.fnv);
    return "{\"elements\": " + std::to_string(c.n) + ", \"mean\": " + json_num(c.mean) + ", \"std\": " +
           json_num(c.std) + ", \"nonfinite\": " + std::to_string(c.nonfinite) + ", \"fnv64\": " + buf + "}";
}

class Session {
public:
    explicit Session(const Args& a) : args(a), plan_only(a.flag("plan-only", false)), rt(plan_only ? -1 : 0), scope(rt) {
        dev.be = rt.backend();
        // --alloc node-order: node memory placed as ggml_gallocr places it
        // (node order, in place where allowed); the executor checks its
        // fusion plan against those addresses.
        const std::string alloc = a.str("alloc", "fused");
        if (alloc == "node-order") rt.set_allocation(HipRuntime::Allocation::NodeOrder);
        else if (alloc != "fused") throw std::runtime_error("--alloc must be fused or node-order");
    }

    Tensor input(const std::string& key) {
        Blob b = read_blob(args.str(key));
        Tensor t = Tensor::empty(b.shape, b.type);
        rt.set_input(*t);
        rt.bind(*t, b.bytes.data(), b.bytes.size());
        return t;
    }
    void param(const Tensor& p, const std::string& key) {
        Blob b = read_blob(args.str("param-" + key));
        if (b.type != DT_TYPE_F32) throw std::runtime_error("parameters are F32");
        if (p.dtype() == DT_TYPE_CONV2D_PACKED) {
            if (!plan_only) pack_conv_weight(p, b);
            return;
        }
        rt.bind(*p, b.bytes.data(), b.bytes.size());
    }
    // A Conv2d weight [Co, Ci, K, K] from fp32 values, packed once on the
    // device into the layout dt_conv2d reads, in a buffer the weight keeps.
    void pack_conv_weight(const Tensor& p, const Blob& b) {
        const Tensor::Shape& s = p.shape();
        const int64_t Co = s[0], Ci = s[1], K = s[2];
        if (b.shape != s || b.bytes.size() != (size_t)(Co * Ci * K * K * 4))
            throw std::runtime_error("packed conv weight: shape mismatch");
        dt_tensor tmp{};
        tmp.type = DT_TYPE_F32;
        tmp.ne[0] = tmp.ne[1] = K;
        tmp.ne[2] = Ci;
        tmp.ne[3] = Co;
        tmp.nb[0] = 4;
        tmp.nb[1] = K * 4;
        tmp.nb[2] = K * K * 4;
        tmp.nb[3] = Ci * K * K * 4;
        tmp.data = dev.alloc(b.bytes.size());
        check(dt_tensor_set(&tmp, b.bytes.data(), 0, b.bytes.size(), nullptr), "dt_tensor_set");
        void* dst = dev.alloc(dt_conv2d_packed_bytes(Co, Ci, K));
        check(dt_conv2d_pack_weights(tmp.data, DT_TYPE_F32, Co, Ci, K, dst, nullptr), "dt_conv2d_pack_weights");
        check(dt_backend_synchronize(rt.backend()), "dt_backend_synchronize");
        dev.release(tmp.data);
        rt.bind_device(*p, dst);
    }
    // An input converted to `type` on the host (e.g. F32 files for BF16 graphs).
    Tensor input_as(const std::string& key, int32_t type) {
        Blob b = read_blob(args.str(key));
        Tensor t = Tensor::empty(b.shape, type);
        rt.set_input(*t);
        auto bytes = convert_blob(b, type);
        rt.bind(*t, bytes.data(), bytes.size());
        return t;
    }
    void output(Tensor t, const std::string& key) {
        if (!t.is_contiguous()) t = t.contiguous();
        rt.set_output(*t);
        outs.push_back({t, args.str(key)});
    }
    // An output summarised in the printed line (element count, moments,
    // FNV-1a of the bytes) instead of written to a file.
    void keep(Tensor t) {
        if (!t.is_contiguous()) t = t.contiguous();
        rt.set_output(*t);
        kept.push_back(t);
    }
    // Every parameter of `m` from DIR/<dotted name>.dtb, converted to the
    // parameter's type.
    void load_weights(const Module& m, const std::string& dir) {
        std::vector<std::pair<std::string, Tensor>> ps;
        m.named_parameters(ps);
        for (auto& p : ps) bind_weight(p.second, read_blob(dir + "/" + p.first + ".dtb"), p.first);
    }
    // --random-weights SEED for the VAE modules: every parameter drawn
    // N(mean, std) in fp32 on the host (mt19937_64), with mean 1 for the
    // GroupNorm weights and 0 otherwise, then bound as a file's values are.
    void random_weights(const Module& m, uint64_t seed, float std) {
        std::vector<std::pair<std::string, Tensor>> ps;
        m.named_parameters(ps);
        std::mt19937_64 gen(seed);
        for (auto& p : ps) {
            // a GroupNorm weight: <prefix.>norm*.weight
            const size_t dot = p.first.rfind('.', p.first.size() - 8);
            const size_t leaf = dot == std::string::npos ? 0 : dot + 1;
            const bool norm_w = p.first.size() > 7 && p.first.compare(p.first.size() - 7, 7, ".weight") == 0 &&
                                p.first.compare(leaf, 4, "norm") == 0;
            std::normal_distribution<float> nd(norm_w ? 1.0f : 0.0f, std);
            Blob b;
            b.shape = p.second.shape();
            b.bytes.resize((size_t)p.second.numel() * 4);
            float* f = reinterpret_cast<float*>(b.bytes.data());
            for (int64_t i = 0; i < p.second.numel(); ++i) f[i] = nd(gen);
            bind_weight(p.second, b, p.first);
        }
    }
    void bind_weight(const Tensor& t, const Blob& b, const std::string& name) {
        if (b.shape != t.shape()) throw std::runtime_error("shape mismatch for " + name);
        if (t.dtype() == DT_TYPE_Q8_0_SPLIT) {
            load_q8_weight(t, b, name);
            return;
        }
        if (t.dtype() == DT_TYPE_CONV2D_PACKED) {
            if (b.type != DT_TYPE_F32) throw std::runtime_error("conv weight " + name + ": F32 expected");
            if (!plan_only) pack_conv_weight(t, b);
            return;
        }
        auto bytes = convert_blob(b, t.dtype());
        if (args.flag("resident-weights", false)) {  // uploaded once, kept in HBM
            void* d = dev.alloc(bytes.size());
            dt_tensor tmp = **t;
            tmp.data = d;
            check(dt_tensor_set(&tmp, bytes.data(), 0, bytes.size(), nullptr), "dt_tensor_set");
            rt.bind_device(*t, d);
        } else {
            rt.bind(*t, bytes.data(), bytes.size());
        }
    }
    // --random-inputs SEED: an N(0, 1) input of `shape` drawn on the host
    // (mt19937_64), stored as `type` and kept resident.
    Tensor random_input(const Tensor::Shape& shape, int32_t type, uint64_t seed) {
        Blob b;
        b.shape = shape;
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        b.bytes.resize((size_t)n * 4);
        float* f = reinterpret_cast<float*>(b.bytes.data());
        std::mt19937_64 gen(seed);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        for (int64_t i = 0; i < n; ++i) f[i] = nd(gen);
        Tensor t = Tensor::empty(shape, type);
        rt.set_input(*t);
        auto bytes = convert_blob(b, type);
        if (!plan_only) {
            void* d = dev.alloc(bytes.size());
            rt.bind_device(*t, d);
            check(dt_tensor_set(*t, bytes.data(), 0, bytes.size(), nullptr), "dt_tensor_set");
        }
        return t;
    }
    // A Q8_0_SPLIT Linear weight from fp32 values: quantised to Q8_0 and
    // repacked on the device into a buffer the weight keeps.
    void load_q8_weight(const Tensor& t, const Blob& b, const std::string& name) {
        if (b.type != DT_TYPE_F32 || t.ndim() != 2 || t.shape()[1] % 32)
            throw std::runtime_error("Q8_0 weight " + name + ": needs F32 rows of a multiple of 32");
        const int64_t rows = t.shape()[0], cols = t.shape()[1];
        void* f32 = dev.alloc((size_t)(rows * cols * 4));
        void* q8 = dev.alloc((size_t)(rows * (cols / 32) * 34));
        dt_tensor tmp{};
        tmp.type = DT_TYPE_F32;
        tmp.ne[0] = cols;
        tmp.ne[1] = rows;
        tmp.ne[2] = tmp.ne[3] = 1;
        tmp.nb[0] = 4;
        tmp.nb[1] = cols * 4;
        tmp.nb[2] = tmp.nb[3] = rows * cols * 4;
        tmp.data = f32;
        check(dt_tensor_set(&tmp, b.bytes.data(), 0, b.bytes.size(), nullptr), "dt_tensor_set");
        void* dst = dev.alloc((size_t)dt_q8_0_split_bytes(rows, cols));
        q8_split_from_f32((const float*)f32, rows, cols, q8, dst);
        check(dt_backend_synchronize(rt.backend()), "dt_backend_synchronize");
        dev.release(q8);
        dev.release(f32);
        rt.bind_device(*t, dst);
    }
    // --plan-only: record and plan the graph without a device.
    void print_plan() {
        const ComputeStats& s = rt.plan();
        std::printf("{\"command\": \"%s\", \"plan_only\": true, \"nodes\": %d, \"fused_nodes\": %d, "
                    "\"mul_mat_nodes\": %d, \"attention_nodes\": %d, \"arena_bytes\": %zu, "
                    "\"naive_bytes\": %zu}\n",
                    args.command.c_str(), s.nodes, s.fused_nodes, s.mul_mat_nodes, s.attention_nodes,
                    s.arena_bytes, s.naive_bytes);
    }
    // --warmup W --steps K: the recorded graph runs W + K times; the median
    // wall time of the last K (each ending in a device synchronisation) is
    // reported as ms_per_compute_median.
    void run() {
        if (plan_only) {
            print_plan();
            return;
        }
        const int steps = (int)std::max<int64_t>(1, args.i64("steps", 1)), warmup = (int)args.i64("warmup", 0);
        std::vector<double> ms;
        for (int i = 0; i < warmup + steps; ++i) {
            const auto t0 = std::chrono::steady_clock::now();
            rt.compute();
            const auto t1 = std::chrono::steady_clock::now();
            if (i >= warmup) ms.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
        }
        std::sort(ms.begin(), ms.end());
        for (auto& o : outs) {
            std::vector<uint8_t> host(HipRuntime::nbytes(*o.first));
            rt.read(*o.first, host.data(), host.size());
            write_blob(o.second, o.first.dtype(), o.first.shape(), host);
        }
        std::string summary;
        for (const Tensor& t : kept) {
            std::vector<uint8_t> host(HipRuntime::nbytes(*t));
            rt.read(*t, host.data(), host.size());
            summary += (summary.empty() ? ", \"output\": " : ", \"output_" + std::to_string(&t - kept.data()) + "\": ") +
                       output_json(check_output(host, t.dtype()));
        }
        const ComputeStats& s = rt.stats();
        std::printf("{\"command\": \"%s\", \"nodes\": %d, \"kernels\": %d, \"fused_nodes\": %d, "
                    "\"arena_bytes\": %zu, \"naive_bytes\": %zu, \"steps\": %d, \"ms_per_compute_median\": %.4f%s}\n",
                    args.command.c_str(), s.nodes, s.kernels, s.fused_nodes, s.arena_bytes, s.naive_bytes, steps,
                    ms[ms.size() / 2], summary.c_str());
    }

    const Args& args;
    bool plan_only;
    HipRuntime rt;
    RuntimeScope scope;
    DeviceBuffers dev;  // after rt: freed before the backend
    std::vector<std::pair<Tensor, std::string>> outs;
    std::vector<Tensor> kept;
};

// ---- Flux2Transformer2DModel: one denoising step --------------------------
//
// Weights come from --weights DIR (one .dtb per parameter), from --gguf PATH
// (a FLUX.2 GGUF checkpoint, fused tensors split as the reference's loader
// splits them) or, with --random-weights SEED, are generated on the device: every Linear weight is
// drawn N(0, 0.02) in fp32 and quantised to Q8_0 (the bytes a GGUF file would
// hold); RMSNorm weights are N(1, 0.02).  --weight-format picks what the GEMMs
// read: bf16 (default; Q8_0 dequantised once to a BF16 copy, 2 bytes per
// weight) or q8_0 (repacked once into DT_TYPE_Q8_0_SPLIT, 1.125 bytes per
// weight, dequantised inside the GEMM to the same bf16 values; weights from
// --weights DIR are quantised on the device first).  Inputs come from files
// or, with --random-inputs SEED, are drawn N(0, 1) (latents, text) with the
// pipeline's position ids (Flux2KleinPipeline.cpp:27-72): text [0, 0, 0, l],
// image [0, y, x, 0] on a square grid.  Inputs and weights are
// device-resident before the first step; --warmup W and --steps K run the
// recorded graph W + K times and report the per-step wall time of the last K.


// Upload host bytes once into a device buffer that `leaf` keeps.
void resident_input(HipRuntime& rt, DeviceBuffers& bufs, const Tensor& leaf, const void* host, size_t bytes) {
    void* d = bufs.alloc(bytes);
    rt.bind_device(*leaf, d);
    check(dt_tensor_set(*leaf, host, 0, bytes, nullptr), "dt_tensor_set");
}

// --hash-weights SEED: weights whose exact values follow from integer
// arithmetic alone, so a host-side check can regenerate them bit for bit
// (the device's libm plays no part).  For a parameter path P:
//   key = splitmix64(SEED * G ^ fnv1a64(P)), z(i) = splitmix64(key + i * G),
//   G = 0x9E3779B97F4A7C15.
// Linear weight [rows, cols]: Q8_0 block b (row-major) has the fp16 scale
// 0x0E00 | (z(9b) & 0x1FF) and codes 4(k-1)+m = (y[2m] + y[2m+1] - 255) / 2
// (truncated) from the bytes y of z(9b+k), k = 1..8, m = 0..3.
// RMSNorm weight i: 1 + ((z(i) >> 40) - 2^23) * 2^-28 in fp32.
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t hash_key(uint64_t seed, const std::string& path) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (unsigned char c : path) h = (h ^ c) * 1099511628211ull;
    return mix64(seed * kGolden ^ h);
}

float hash_norm_weight(uint64_t key, int64_t i) {
    return 1.0f + (float)((int32_t)(mix64(key + (uint64_t)i * kGolden) >> 40) - 8388608) * 0x1.0p-28f;
}

void hash_q8_0_blocks(uint64_t key, int64_t n_blocks, uint8_t* out) {
    const unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < nt; ++t)
        pool.emplace_back([=] {
            for (int64_t b = (int64_t)t; b < n_blocks; b += nt) {
                uint8_t* blk = out + b * 34;
                const uint32_t d = 0x0E00u | (uint32_t)(mix64(key + (uint64_t)(9 * b) * kGolden) & 0x1FF);
                blk[0] = (uint8_t)d;
                blk[1] = (uint8_t)(d >> 8);
                for (int k = 1; k <= 8; ++k) {
                    const uint64_t z = mix64(key + (uint64_t)(9 * b + k) * kGolden);
                    for (int m = 0; m < 4; ++m) {
                        const int sum = (int)((z >> (16 * m)) & 0xFF) + (int)((z >> (16 * m + 8)) & 0xFF);
                        blk[2 + 4 * (k - 1) + m] = (uint8_t)(int8_t)((sum - 255) / 2);
                    }
                }
            }
        });
    for (auto& th : pool) th.join();
}

// Every Linear weight of m drawn (device N(0, 0.02), quantised to Q8_0 there)
// or hash-drawn as Q8_0 blocks on the host, then kept as a BF16 copy or in
// the DT_TYPE_Q8_0_SPLIT layout; RMSNorm weights N(1, 0.02) or hash-drawn.
void random_weights(HipRuntime& rt, const Module& m, uint64_t seed, bool hashed, DeviceBuffers& bufs,
                    size_t* resident_bytes, size_t* q8_bytes, size_t* n_params) {
    std::vector<std::pair<std::string, Tensor>> ps;
    m.named_parameters(ps);
    auto linear = [](const Tensor& t) {
        return t.dtype() == DT_TYPE_BF16 || t.dtype() == DT_TYPE_Q8_0_SPLIT || (t.dtype() == DT_TYPE_F32 && t.ndim() == 2);
    };
    auto resident = [](const Tensor& t) {
        return t.dtype() == DT_TYPE_BF16  ? (size_t)t.numel() * 2
               : t.dtype() == DT_TYPE_F32 ? (size_t)t.numel() * 4
                                          : (size_t)dt_q8_0_split_bytes(t.shape()[0], t.shape()[1]);
    };
    size_t total = 0, max_n = 0;
    for (auto& p : ps)
        if (linear(p.second)) {
            if (p.second.ndim() != 2 || p.second.shape()[1] % 32)
                throw std::runtime_error("random weight layout: " + p.first);
            total += align256(resident(p.second));
            max_n = std::max(max_n, (size_t)p.second.numel());
        }
    char* big = (char*)bufs.alloc(total);
    float* f32 = hashed ? nullptr : (float*)bufs.alloc(max_n * 4);
    void* q8 = bufs.alloc(max_n / 32 * 34 + 256);
    std::vector<uint8_t> host_q8(hashed ? max_n / 32 * 34 : 0);
    std::mt19937_64 gen(seed);
    std::normal_distribution<float> nd(1.0f, 0.02f);
    size_t off = 0, idx = 0;
    *resident_bytes = *q8_bytes = *n_params = 0;
    for (auto& p : ps) {
        const Tensor& t = p.second;
        *n_params += (size_t)t.numel();
        ++idx;
        if (linear(t)) {
            const int64_t rows = t.shape()[0], cols = t.shape()[1], rb = cols / 32 * 34;
            if (hashed) {
                hash_q8_0_blocks(hash_key(seed, p.first), rows * (cols / 32), host_q8.data());
                dt_tensor blocks{};  // the Q8_0 bytes as a [rows, cols] Q8_0 tensor
                blocks.type = DT_TYPE_Q8_0;
                blocks.ne[0] = cols;
                blocks.ne[1] = rows;
                blocks.ne[2] = blocks.ne[3] = 1;
                blocks.nb[0] = 34;
                blocks.nb[1] = rb;
                blocks.nb[2] = blocks.nb[3] = rb * rows;
                blocks.data = q8;
                check(dt_tensor_set(&blocks, host_q8.data(), 0, (size_t)(rows * rb), nullptr), "dt_tensor_set");
            } else {
                check(dt_fill_randn(f32, rows * cols, seed * 1000003ull + idx, 0.0f, 0.02f, nullptr),
                      "dt_fill_randn");
                check(dt_quantize_q8_0(f32, rows, cols, cols, q8, rb, nullptr), "dt_quantize_q8_0");
            }
            if (t.dtype() == DT_TYPE_BF16 || t.dtype() == DT_TYPE_F32) {
                check(dt_dequant(q8, DT_TYPE_Q8_0, rows, cols, rb, big + off, cols, t.dtype(), nullptr),
                      "dt_dequant");
            } else {
                check(dt_q8_0_split(q8, rows, cols, rb, big + off, cols,
                                    reinterpret_cast<float*>(big + off + dt_q8_0_split_scale_offset(rows, cols)),
                                    rows, nullptr),
                      "dt_q8_0_split");
            }
            rt.bind_device(*t, big + off);
            off += align256(resident(t));
            *resident_bytes += resident(t);
            *q8_bytes += (size_t)(rows * rb);
        } else if (t.dtype() == DT_TYPE_F32 && t.ndim() == 1) {
            std::vector<float> h((size_t)t.numel());
            if (hashed) {
                const uint64_t key = hash_key(seed, p.first);
                for (size_t i = 0; i < h.size(); ++i) h[i] = hash_norm_weight(key, (int64_t)i);
            } else {
                for (float& v : h) v = nd(gen);  // RMSNorm weights
            }
            resident_input(rt, bufs, t, h.data(), h.size() * 4);
        } else {
            throw std::runtime_error("random weights: unexpected parameter type for " + p.first);
        }
    }
}

// Count of each recorded op (unary ops by kind), as a JSON object: the op
// set a ggml-side translation of the same graph has to map.
std::string op_histogram(const HipRuntime& rt) {
    static const char* kOps[] = {"NONE", "ADD", "SUB", "MUL", "DIV", "SCALE", "SIGMOID", "NORM", "RMS_NORM",
                                 "ROPE", "CONCAT", "CPY", "VIEW", "FILL", "UNARY", "MUL_MAT", "FLASH_ATTN_EXT",
                                 "CONV_2D_DIRECT", "UPSCALE"};
    static const char* kUnary[] = {"SIGMOID", "EXP", "LOG", "SQRT", "SIN", "COS", "SCALE", "CLAMP", "SILU",
                                   "FILL"};
    std::map<std::string, int> h;
    for (const Node* t : rt.nodes()) {
        std::string name = t->op >= 0 && t->op < (int)(sizeof kOps / sizeof *kOps) ? kOps[t->op] : "?";
        if (t->op == DT_OP_UNARY) {
            const int k = t->op_params[0];
            name += std::string(".") + (k >= 0 && k < (int)(sizeof kUnary / sizeof *kUnary) ? kUnary[k] : "?");
        }
        ++h[name];
    }
    std::string out = "{";
    for (const auto& kv : h) out += (out.size() > 1 ? ", " : "") + json_str(kv.first) + ": " + std::to_string(kv.second);
    return out + "}";
}

void run_model(Session& s, const Args& a) {
    Flux2Config cfg;
    cfg.num_layers = a.i64("num_layers", 5);
    cfg.num_single_layers = a.i64("num_single_layers", 20);
    cfg.num_attention_heads = a.i64("num_attention_heads", 24);
    cfg.attention_head_dim = a.i64("attention_head_dim", 128);
    cfg.in_channels = cfg.out_channels = a.i64("in_channels", 128);
    cfg.joint_attention_dim = a.i64("joint_attention_dim", 2560);
    cfg.mlp_ratio = a.f32("mlp_ratio", 3.0f);
    cfg.rope_theta = a.i64("rope_theta", 2000);
    cfg.guidance_embeds = a.flag("guidance_embeds", false);
    if (a.has("axes_dims_rope")) cfg.axes_dims_rope = a.list("axes_dims_rope");
    const int64_t n_img = a.i64("img_tokens", 4096), n_txt = a.i64("txt_tokens", 512);
    const int steps = (int)a.i64("steps", 1), warmup = (int)a.i64("warmup", 0);

    HipRuntime& rt = s.rt;
    DeviceBuffers& bufs = s.dev;
    const std::string format = a.str("weight-format", "bf16");
    if (format != "bf16" && format != "q8_0" && format != "f32")
        throw std::runtime_error("--weight-format must be bf16, q8_0 or f32");
    LinearWeightType wt(format == "q8_0" ? DT_TYPE_Q8_0_SPLIT : format == "f32" ? DT_TYPE_F32 : DT_TYPE_BF16);
    // --dtype: the activations' type (bf16, or f32 as the reference keeps them)
    const std::string dtype = a.str("dtype", "bf16");
    if (dtype != "bf16" && dtype != "f32") throw std::runtime_error("--dtype must be bf16 or f32");
    const int32_t act = dtype == "f32" ? DT_TYPE_F32 : DT_TYPE_BF16;
    Flux2Transformer2DModel model(cfg);

    Tensor hidden = Tensor::empty({1, n_img, cfg.in_channels}, act);
    Tensor text = Tensor::empty({1, n_txt, cfg.joint_attention_dim}, act);
    Tensor timestep = Tensor::empty({1}, DT_TYPE_F32);
    Tensor img_ids = Tensor::empty({n_img, 4}, DT_TYPE_I32);
    Tensor txt_ids = Tensor::empty({n_txt, 4}, DT_TYPE_I32);
    for (const Tensor* t : {&hidden, &text, &timestep, &img_ids, &txt_ids}) rt.set_input(**t);

    size_t resident_bytes = 0, q8_bytes = 0, n_params = 0;
    if (s.plan_only && a.has("gguf")) {
        // Where each parameter would be read from (no device): the file
        // tensor, rows or columns, and the range; then the unused tensors.
        GgufFile f(a.str("gguf"));
        std::vector<std::pair<std::string, Tensor>> ps;
        model.named_parameters(ps);
        std::map<std::string, std::vector<int64_t>> shapes;
        for (auto& p : ps) shapes[p.first] = p.second.shape();
        std::map<std::string, int> used;
        std::string out = "{\"command\": \"Flux2Transformer2DModel\", \"gguf_plan\": {";
        for (size_t i = 0; i < ps.size(); ++i) {
            const GgufSource src = gguf_source(f, ps[i].first, shapes);
            used[src.tensor->name] = 1;
            out += std::string(i ? ", " : "") + json_str(ps[i].first) + ": [" + json_str(src.tensor->name) + ", \"" +
                   (src.by_cols ? "cols" : "rows") + "\", " + std::to_string(src.begin) + ", " +
                   std::to_string(src.end) + "]";
        }
        out += "}, \"unused\": [";
        bool first = true;
        for (const GgufTensor& t : f.tensors())
            if (!used.count(t.name)) {
                out += (first ? "" : ", ") + json_str(t.name);
                first = false;
            }
        out += "]}";
        std::printf("%s\n", out.c_str());
        return;
    }
    if (s.plan_only) {
        std::vector<std::pair<std::string, Tensor>> ps;
        model.named_parameters(ps);
        for (auto& p : ps) n_params += (size_t)p.second.numel();
        Tensor out = model.forward(hidden, text, timestep, img_ids, txt_ids);
        rt.set_output(*out);
        const ComputeStats& st = rt.plan();
        std::printf("{\"command\": \"Flux2Transformer2DModel\", \"plan_only\": true, \"nodes\": %d, "
                    "\"fused_nodes\": %d, \"grouped_nodes\": %d, \"deferred_nodes\": %d, "
                    "\"mul_mat_nodes\": %d, \"attention_nodes\": %d, "
                    "\"arena_bytes\": %zu, \"naive_bytes\": %zu, \"params\": %zu, \"alloc\": \"%s\", "
                    "\"launches_held\": %d, \"fused_nodes_checked\": %d, \"ops\": %s}\n",
                    st.nodes, st.fused_nodes, st.grouped_nodes, st.deferred_nodes, st.mul_mat_nodes,
                    st.attention_nodes, st.arena_bytes, st.naive_bytes, n_params, a.str("alloc", "fused").c_str(),
                    st.launches_held, st.fused_nodes_checked, op_histogram(rt).c_str());
        return;
    }
    std::string gguf_note;
    if (a.has("random-weights") || a.has("hash-weights")) {
        const bool hashed = a.has("hash-weights");
        random_weights(rt, model, (uint64_t)a.i64(hashed ? "hash-weights" : "random-weights"), hashed, bufs,
                       &resident_bytes, &q8_bytes, &n_params);
    } else if (a.has("gguf")) {
        // A GGUF checkpoint, placed as the reference's GGUFLoaderVisitor
        // reads it (fused q/k/v/mlp, to_out and linear_in tensors split).
        GgufFile f(a.str("gguf"));
        const GgufLoadStats st = load_gguf(model, f, rt, [&](size_t n) { return bufs.alloc(n); });
        gguf_note = ", \"gguf_tensors_used\": " + std::to_string(st.file_tensors_used) +
                    ", \"gguf_tensors_unused\": " + std::to_string(st.unused.size()) +
                    ", \"gguf_bytes_read\": " + std::to_string(st.bytes_read);
        std::vector<std::pair<std::string, Tensor>> ps;
        model.named_parameters(ps);
        for (auto& p : ps) n_params += (size_t)p.second.numel();
    } else {
        s.load_weights(model, a.str("weights"));
    }

    if (a.has("random-inputs")) {
        std::mt19937_64 gen((uint64_t)a.i64("random-inputs"));
        std::normal_distribution<float> nd(0.0f, 1.0f);
        auto bf16_normals = [&](int64_t n) {
            std::vector<uint16_t> v((size_t)n);
            for (auto& x : v) x = f32_to_bf16(nd(gen));
            return v;
        };
        auto h = bf16_normals(hidden.numel()), e = bf16_normals(text.numel());
        auto upload = [&](const Tensor& t, const std::vector<uint16_t>& v) {  // the same values in either type
            if (act == DT_TYPE_BF16) return resident_input(rt, bufs, t, v.data(), v.size() * 2);
            std::vector<float> f(v.size());
            for (size_t i = 0; i < v.size(); ++i) {
                const uint32_t u = (uint32_t)v[i] << 16;
                std::memcpy(&f[i], &u, 4);
            }
            resident_input(rt, bufs, t, f.data(), f.size() * 4);
        };
        upload(hidden, h);
        upload(text, e);
        const float ts = a.f32("timestep", 0.5f);
        resident_input(rt, bufs, timestep, &ts, 4);
        const int64_t side = (int64_t)std::llround(std::sqrt((double)n_img));
        if (side * side != n_img) throw std::runtime_error("--img_tokens must be a square for random inputs");
        std::vector<int32_t> ii((size_t)n_img * 4, 0), ti((size_t)n_txt * 4, 0);
        for (int64_t y = 0; y < side; ++y)
            for (int64_t x = 0; x < side; ++x) {
                ii[(size_t)(y * side + x) * 4 + 1] = (int32_t)y;
                ii[(size_t)(y * side + x) * 4 + 2] = (int32_t)x;
            }
        for (int64_t l = 0; l < n_txt; ++l) ti[(size_t)l * 4 + 3] = (int32_t)l;
        resident_input(rt, bufs, img_ids, ii.data(), ii.size() * 4);
        resident_input(rt, bufs, txt_ids, ti.data(), ti.size() * 4);
    } else {
        auto bind_file = [&](const Tensor& t, const std::string& key) {
            Blob b = read_blob(a.str(key));
            auto bytes = convert_blob(b, t.dtype());
            if (b.shape != t.shape()) throw std::runtime_error("input shape mismatch for " + key);
            rt.bind(*t, bytes.data(), bytes.size());
        };
        bind_file(hidden, "hidden_states");
        bind_file(text, "encoder_hidden_states");
        bind_file(timestep, "timestep");
        bind_file(img_ids, "img_ids");
        bind_file(txt_ids, "txt_ids");
    }

    Tensor out = model.forward(hidden, text, timestep, img_ids, txt_ids);
    if (!out.is_contiguous()) out = out.contiguous();
    rt.set_output(*out);

    // --hip-graph true: the step is recorded once and replayed as a HIP graph.
    // --replan true: the device-less plan (HipRuntime::plan) runs between
    // steps, as a caller inspecting the placement would; the steps' output
    // must not change.
    const bool replay = a.flag("hip-graph", false), replan = a.flag("replan", false);
    std::vector<double> ms;
    for (int i = 0; i < warmup + steps; ++i) {
        if (replan && i > 0) rt.plan();
        const auto t0 = std::chrono::steady_clock::now();
        if (replay)
            rt.compute_graph();
        else
            rt.compute();
        const auto t1 = std::chrono::steady_clock::now();
        if (i >= warmup) ms.push_back(std::chrono::duration<double, std::milli>(t1 - t0).count());
    }
    std::vector<uint8_t> host(HipRuntime::nbytes(*out));
    rt.read(*out, host.data(), host.size());
    if (a.has("out")) write_blob(a.str("out"), out.dtype(), out.shape(), host);
    const OutputCheck oc = check_output(host, out.dtype());
    std::vector<double> sorted = ms;
    std::sort(sorted.begin(), sorted.end());
    double mean = 0;
    for (double v : ms) mean += v;
    mean /= std::max<size_t>(ms.size(), 1);
    const ComputeStats& st = rt.stats();
    std::printf("{\"command\": \"Flux2Transformer2DModel\", \"steps\": %d, \"warmup\": %d, "
                "\"ms_per_step_median\": %.4f, \"ms_per_step_mean\": %.4f, \"ms_per_step_min\": %.4f, "
                "\"nodes\": %d, \"kernels\": %d, \"fused_nodes\": %d, \"arena_bytes\": %zu, "
                "\"params\": %zu, \"weight_format\": \"%s\", \"linear_weight_bytes\": %zu, "
                "\"q8_0_weight_bytes\": %zu, \"hip_graph\": %s, \"alloc\": \"%s\", \"gemm\": \"%s\", "
                "\"launches_held\": %d, \"output\": %s%s}\n",
                steps, warmup, sorted.empty() ? 0.0 : sorted[sorted.size() / 2], mean,
                sorted.empty() ? 0.0 : sorted.front(), st.nodes, st.kernels, st.fused_nodes, st.arena_bytes,
                n_params, format.c_str(), resident_bytes, q8_bytes, replay ? "true" : "false",
                a.str("alloc", "fused").c_str(), "mfma", st.launches_held,
                output_json(oc).c_str(), gguf_note.c_str());
    std::fflush(stdout);
    if (oc.nonfinite)
        throw std::runtime_error("the step's output holds " + std::to_string(oc.nonfinite) + " non-finite values");
}

// GgufInfo --gguf PATH: the file's header, metadata and tensor table as one
// JSON line (no device needed).
void gguf_info(const Args& a) {
    GgufFile f(a.str("gguf"));
    std::string out = "{\"command\": \"GgufInfo\", \"path\": " + json_str(f.path()) +
                      ", \"version\": " + std::to_string(f.version()) +
                      ", \"alignment\": " + std::to_string(f.alignment()) +
                      ", \"data_offset\": " + std::to_string(f.data_offset()) +
                      ", \"file_size\": " + std::to_string(f.file_size()) + ", \"metadata\": {";
    bool first = true;
    for (const auto& kv : f.metadata()) {
        const GgufValue& v = kv.second;
        out += (first ? "" : ", ") + json_str(kv.first) + ": ";
        first = false;
        if (v.type == 8) {
            out += json_str(v.s);
        } else if (v.type == 9) {
            out += "{\"array_type\": " + std::to_string(v.array_type) + ", \"count\": " +
                   std::to_string(v.array_count) + ", \"values\": [";
            if (v.array_type == 8)
                for (size_t i = 0; i < v.array_strings.size(); ++i) out += (i ? ", " : "") + json_str(v.array_strings[i]);
            else
                for (size_t i = 0; i < v.array_numbers.size(); ++i) out += (i ? ", " : "") + json_num(v.array_numbers[i]);
            out += "]}";
        } else if (v.type == 10) {
            out += std::to_string(v.u);
        } else if (v.type == 11) {
            out += std::to_string(v.i);
        } else {
            out += json_num(v.f);
        }
    }
    out += "}, \"tensors\": [";
    for (size_t i = 0; i < f.tensors().size(); ++i) {
        const GgufTensor& t = f.tensors()[i];
        out += std::string(i ? ", " : "") + "{\"name\": " + json_str(t.name) + ", \"type\": " +
               std::to_string(t.type) + ", \"type_name\": \"" + ggml_type_label(t.type) + "\", \"ne\": [";
        for (int d = 0; d < t.n_dims; ++d) out += (d ? ", " : "") + std::to_string(t.ne[d]);
        out += "], \"offset\": " + std::to_string(t.offset) + ", \"nbytes\": " + std::to_string(t.nbytes) + "}";
    }
    out += "]}";
    std::printf("%s\n", out.c_str());
}

// HashWeights: the host-side values of --hash-weights for one parameter.
void hash_weights(const Args& a) {
    const uint64_t seed = (uint64_t)a.i64("seed");
    const std::string path = a.str("path");
    const int64_t rows = a.i64("rows"), cols = a.i64("cols", 0);
    std::vector<uint8_t> bytes;
    if (cols) {
        if (rows <= 0 || cols % 32) throw std::runtime_error("HashWeights: rows > 0 and cols % 32 == 0");
        bytes.resize((size_t)(rows * (cols / 32) * 34));
        hash_q8_0_blocks(hash_key(seed, path), rows * (cols / 32), bytes.data());
    } else {
        const uint64_t key = hash_key(seed, path);
        std::vector<float> w((size_t)rows);
        for (int64_t i = 0; i < rows; ++i) w[i] = hash_norm_weight(key, i);
        bytes.resize(w.size() * 4);
        std::memcpy(bytes.data(), w.data(), bytes.size());
    }
    std::ofstream f(a.str("out"), std::ios::binary);
    f.write(reinterpret_cast<const char*>(bytes.data()), (std::streamsize)bytes.size());
    if (!f) throw std::runtime_error("HashWeights: cannot write " + a.str("out"));
    std::printf("{\"command\": \"HashWeights\", \"bytes\": %zu}\n", bytes.size());
}

void run(const Args& a) {
    if (a.command == "GgufInfo") {
        gguf_info(a);
        return;
    }
    if (a.command == "HashWeights") {
        hash_weights(a);
        return;
    }
    Session s(a);
    const std::string& c = a.command;
    if (c == "LayerNorm") {
        LayerNorm m(a.i64("dim"), a.f32("eps", 1e-5f), a.flag("elementwise_affine", true), a.flag("bias", true));
        Tensor x = s.input("x");
        if (a.flag("elementwise_affine", true)) {
            s.param(m.weight, "weight");
            if (a.flag("bias", true)) s.param(m.bias, "bias");
        }
        s.output(m.forward(x), "out");
    } else if (c == "RMSNorm") {
        RMSNorm m(a.i64("dim"), a.f32("eps", 1e-5f), a.flag("elementwise_affine", true));
        Tensor x = s.input("x");
        if (a.flag("elementwise_affine", true)) s.param(m.weight, "weight");
        s.output(m.forward(x), "out");
    } else if (c == "GroupNorm") {
        const bool affine = a.flag("affine", true), bias = a.flag("bias", true);
        GroupNorm m(a.i64("num_groups"), a.i64("num_channels"), a.f32("eps", 1e-5f), affine, bias);
        Tensor x = s.input("input");
        if (affine) {
            s.param(m.weight, "weight");
            if (bias) s.param(m.bias, "bias");
        }
        Tensor y = m.forward(x);
        if (a.flag("silu", false)) y = SiLU().forward(y);   // ResnetBlock2D.inl:111-122
        s.output(y, "out");
    } else if (c == "Conv2d") {
        // Conv2d.py: --in_channels, --out_channels, --kernel_size, --stride, --padding, --bias;
        // --packed-weights true packs the weight once at load (DT_TYPE_CONV2D_PACKED)
        const bool bias = a.flag("bias", true);
        ConvWeightType cw(a.flag("packed-weights", false) ? DT_TYPE_CONV2D_PACKED : DT_TYPE_F32);
        Conv2d m(a.i64("in_channels"), a.i64("out_channels"), a.i64("kernel_size"), a.i64("stride", 1),
                 a.i64("padding", 0), bias);
        Tensor x = s.input("x");
        s.param(m.weight, "weight");
        if (bias) s.param(m.bias, "bias");
        s.output(m.forward(x), "out");
    } else if (c == "Upsample2D") {
        // Upsample2D.py: --channels, --use_conv, --out_channels
        const bool use_conv = a.flag("use_conv", false);
        ConvWeightType cw(a.flag("packed-weights", false) ? DT_TYPE_CONV2D_PACKED : DT_TYPE_F32);
        Upsample2D m(a.i64("channels"), use_conv, a.i64("out_channels", -1));
        Tensor x = s.input("hidden_states");
        if (use_conv) {
            s.param(m.conv()->weight, "conv.weight");
            s.param(m.conv()->bias, "conv.bias");
        }
        s.output(m.forward(x), "out");
    } else if (c == "ResnetBlock2D") {
        // ResnetBlock2D.py (the reference CLI's main.cpp:126-170 arguments): --in_channels,
        // --out_channels, --temb_channels, --groups, --groups_out, --eps, --kernel_size,
        // --output_scale_factor, --use_in_shortcut, --conv_shortcut_bias, --conv_2d_out_channels;
        // inputs --hidden_states [--temb]; parameters from --weights DIR (one .dtb per dotted
        // name); --dtype f32|bf16 for the activations; --packed-weights true packs the conv
        // weights once at load
        const int32_t act = a.str("dtype", "f32") == "bf16" ? DT_TYPE_BF16 : DT_TYPE_F32;
        LinearWeightType wt(act);
        ConvWeightType cw(a.flag("packed-weights", false) ? DT_TYPE_CONV2D_PACKED : DT_TYPE_F32);
        auto opt = [&](const char* k) { return a.has(k) ? std::optional<int64_t>(a.i64(k)) : std::nullopt; };
        const std::optional<bool> use_in_shortcut =
            a.has("use_in_shortcut") ? std::optional<bool>(a.flag("use_in_shortcut", false)) : std::nullopt;
        ResnetBlock2D<SiLU> m(a.i64("in_channels"), opt("out_channels"), std::nullopt, 0.0f, opt("temb_channels"),
                              a.i64("groups", 32), opt("groups_out"), true, a.f32("eps", 1e-6f), false,
                              a.i64("kernel_size", 3), a.f32("output_scale_factor", 1.0f), use_in_shortcut, false,
                              false, a.flag("conv_shortcut_bias", true), opt("conv_2d_out_channels"));
        // --random-inputs SEED --batch N --height H --width W [--random-weights SEED]: generated
        // instead of read (no temb); --out is then optional
        Tensor x = a.has("random-inputs")
                       ? s.random_input({a.i64("batch", 1), a.i64("in_channels"), a.i64("height"), a.i64("width")},
                                        act, (uint64_t)a.i64("random-inputs"))
                       : s.input_as("hidden_states", act);
        std::optional<Tensor> temb;
        if (a.has("temb")) temb = s.input_as("temb", act);
        if (a.has("random-weights")) s.random_weights(m, (uint64_t)a.i64("random-weights"), 0.02f);
        else s.load_weights(m, a.str("weights"));
        Tensor y = m.forward(x, temb ? &*temb : nullptr);
        if (a.has("out")) s.output(y, "out");
        else s.keep(y);
    } else if (c == "UpDecoderBlock2D") {
        // UpDecoderBlock2D.py (the reference CLI's main.cpp:461-497 arguments): --in_channels,
        // --out_channels, --num_layers, --resnet_groups, --output_scale_factor, --add_upsample,
        // --temb_channels; --hidden_states, or --random-inputs SEED with --batch --height --width;
        // parameters from --weights DIR or --random-weights SEED; --dtype f32|bf16;
        // --packed-weights true packs the conv weights once at load
        const int32_t act = a.str("dtype", "f32") == "bf16" ? DT_TYPE_BF16 : DT_TYPE_F32;
        LinearWeightType wt(act);
        ConvWeightType cw(a.flag("packed-weights", false) ? DT_TYPE_CONV2D_PACKED : DT_TYPE_F32);
        UpDecoderBlock2D m(a.i64("in_channels"), a.i64("out_channels"), std::nullopt, 0.0f, a.i64("num_layers", 1),
                           1e-6f, a.i64("resnet_groups", 32), true, a.f32("output_scale_factor", 1.0f),
                           a.flag("add_upsample", true),
                           a.has("temb_channels") ? std::optional<int64_t>(a.i64("temb_channels")) : std::nullopt);
        Tensor x = a.has("random-inputs")
                       ? s.random_input({a.i64("batch", 1), a.i64("in_channels"), a.i64("height"), a.i64("width")},
                                        act, (uint64_t)a.i64("random-inputs"))
                       : s.input_as("hidden_states", act);
        if (a.has("random-weights")) s.random_weights(m, (uint64_t)a.i64("random-weights"), 0.02f);
        else s.load_weights(m, a.str("weights"));
        Tensor y = m.forward(x);
        if (a.has("out")) s.output(y, "out");
        else s.keep(y);
    } else if (c == "SiLU") {
        s.output(SiLU().forward(s.input("x")), "out");
    } else if (c == "Flux2PosEmbed") {
        Flux2PosEmbed m(a.i64("theta"), a.list("axes_dim"));
        Tensor x = s.input("x");
        s.output(m.forward(x, s.input("position_ids")), "out");
    } else if (c == "Flux2SwiGLU") {
        Tensor g = s.input("gate");
        s.output(Flux2SwiGLU().forward(g, s.input("up")), "out");
    } else if (c == "AdaLNModulation") {
        // norm -> (1 + scale) * n + shift with shift/scale chunks of a [1, 3*D] modulation
        Tensor x = s.input("x");
        Tensor mod = s.input("mod");
        LayerNorm norm(x.shape().back(), a.f32("eps", 1e-6f), false);
        auto sets = Flux2Modulation::split(mod, 1);
        s.output(adaln_modulate(norm, x, sets[0][0], sets[0][1]), "out");
    } else if (c == "Flux2SingleBlockElementwise") {
        // The elementwise chain of Flux2SingleTransformerBlock / Flux2ParallelSelfAttention
        // around its GEMMs and attention, whose outputs are given as inputs:
        // adaLN of x, QK RMSNorm + Flux2PosEmbed, SwiGLU and the gated residual.
        const int64_t heads = a.i64("heads");
        Tensor x = s.input("x"), mod = s.input("mod");
        Tensor q = s.input("q"), k = s.input("k");
        Tensor gate = s.input("mlp_gate"), up = s.input("mlp_up"), attn = s.input("attn_out");
        Tensor pos = s.input("position_ids");
        const int64_t dim = x.shape().back(), head_dim = dim / heads;
        LayerNorm norm(dim, a.f32("eps", 1e-6f), false);
        RMSNorm norm_q(head_dim, a.f32("eps", 1e-6f)), norm_k(head_dim, a.f32("eps", 1e-6f));
        s.param(norm_q.weight, "norm_q");
        s.param(norm_k.weight, "norm_k");
        Flux2PosEmbed pe(a.i64("theta"), a.list("axes_dim"));
        auto m = Flux2Modulation::split(mod, 1)[0];
        Tensor nx = adaln_modulate(norm, x, m[0], m[1]);
        Tensor qh = pe.forward(norm_q.forward(q.unflatten(-1, {heads, -1})), pos);
        Tensor kh = pe.forward(norm_k.forward(k.unflatten(-1, {heads, -1})), pos);
        Tensor mlp = Flux2SwiGLU().forward(gate, up);
        Tensor res = gated_residual(x, m[2], attn);
        s.output(nx, "out-norm");
        s.output(qh, "out-q");
        s.output(kh, "out-k");
        s.output(mlp, "out-mlp");
        s.output(res, "out-residual");
    } else if (c == "Flux2DoubleStreamQK") {
        // Flux2Attention.hpp:93-122: txt and img q normalised with their own
        // RMSNorm, concatenated txt-first along the sequence, then RoPE.
        const int64_t heads = a.i64("heads");
        Tensor qt = s.input("txt_q"), qi = s.input("img_q"), pos = s.input("position_ids");
        const int64_t head_dim = qt.shape().back() / heads;
        RMSNorm nt(head_dim, a.f32("eps", 1e-6f)), ni(head_dim, a.f32("eps", 1e-6f));
        s.param(nt.weight, "norm_added_q");
        s.param(ni.weight, "norm_q");
        Flux2PosEmbed pe(a.i64("theta"), a.list("axes_dim"));
        Tensor q = Tensor::cat({nt.forward(qt.unflatten(-1, {heads, -1})),
                                ni.forward(qi.unflatten(-1, {heads, -1}))}, 1);
        s.output(pe.forward(q, pos), "out");
    } else if (c == "Flux2SingleTransformerBlock") {
        // Full block (Flux2SingleTransformerBlock.hpp:36-72) with weights from --weights DIR.
        const int32_t act = a.str("dtype", "bf16") == "bf16" ? DT_TYPE_BF16 : DT_TYPE_F32;
        LinearWeightType wt(act == DT_TYPE_BF16 ? DT_TYPE_BF16 : DT_TYPE_F32);
        Tensor x = s.input_as("hidden_states", act);
        Tensor mod = s.input("temb_mod"), pos = s.input("position_ids");
        const int64_t dim = x.shape().back(), heads = a.i64("heads");
        Flux2SingleTransformerBlock block(dim, heads, dim / heads, a.f32("mlp_ratio", 3.0f), a.f32("eps", 1e-6f),
                                          false);
        s.load_weights(block, a.str("weights"));
        Flux2PosEmbed pe(a.i64("theta"), a.list("axes_dim"));
        s.output(block.forward(x, mod, {&pe, pos}), "out");
    } else if (c == "Flux2TransformerBlock") {
        // Double-stream block (Flux2TransformerBlock.hpp:47-116) with weights from --weights DIR.
        const int32_t act = a.str("dtype", "bf16") == "bf16" ? DT_TYPE_BF16 : DT_TYPE_F32;
        LinearWeightType wt(act == DT_TYPE_BF16 ? DT_TYPE_BF16 : DT_TYPE_F32);
        Tensor x = s.input_as("hidden_states", act), e = s.input_as("encoder_hidden_states", act);
        Tensor mi = s.input("temb_mod_img"), mt = s.input("temb_mod_txt"), pos = s.input("position_ids");
        const int64_t dim = x.shape().back(), heads = a.i64("heads");
        Flux2TransformerBlock block(dim, heads, dim / heads, a.f32("mlp_ratio", 3.0f), a.f32("eps", 1e-6f), false);
        s.load_weights(block, a.str("weights"));
        Flux2PosEmbed pe(a.i64("theta"), a.list("axes_dim"));
        auto [enc, hid] = block.forward(x, e, mi, mt, {&pe, pos});
        s.output(enc, "out-encoder");
        s.output(hid, "out-hidden");
    } else if (c == "Flux2Transformer2DModel") {
        run_model(s, a);
        return;
    } else {
        throw std::runtime_error("unknown command " + c);
    }
    s.run();
}

}  // namespace

int main(int argc, char** argv) {
    try {
        run(parse(argc, argv));
    } catch (const std::exception& e) {
        std::fprintf(stderr, "dit_cli: %s\n", e.what());
        return 1;
    }
    return 0;
}
