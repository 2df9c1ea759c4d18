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
// message on stderr and exit non-zero.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "modules.hpp"

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
    b.shape.resize(hdr[2]);
    f.read((char*)b.shape.data(), sizeof(int64_t) * hdr[2]);
    int64_t n = 1;
    for (int64_t d : b.shape) n *= d;
    const int64_t es = (b.type == DT_TYPE_F32 || b.type == DT_TYPE_I32) ? 4 : 2;
    b.bytes.resize((size_t)(n * es));
    f.read((char*)b.bytes.data(), (std::streamsize)b.bytes.size());
    if (!f) throw std::runtime_error("truncated tensor file " + path);
    return b;
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

class Session {
public:
    explicit Session(const Args& a) : args(a), rt(0), scope(rt) {}

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
        rt.bind(*p, b.bytes.data(), b.bytes.size());
    }
    void output(Tensor t, const std::string& key) {
        if (!t.is_contiguous()) t = t.contiguous();
        rt.set_output(*t);
        outs.push_back({t, args.str(key)});
    }
    void run() {
        rt.compute();
        for (auto& o : outs) {
            std::vector<uint8_t> host(HipRuntime::nbytes(*o.first));
            rt.read(*o.first, host.data(), host.size());
            write_blob(o.second, o.first.dtype(), o.first.shape(), host);
        }
        const ComputeStats& s = rt.stats();
        std::printf("{\"command\": \"%s\", \"nodes\": %d, \"kernels\": %d, \"fused_nodes\": %d, "
                    "\"arena_bytes\": %zu, \"naive_bytes\": %zu}\n",
                    args.command.c_str(), s.nodes, s.kernels, s.fused_nodes, s.arena_bytes, s.naive_bytes);
    }

    const Args& args;
    HipRuntime rt;
    RuntimeScope scope;
    std::vector<std::pair<Tensor, std::string>> outs;
};

void run(const Args& a) {
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
