// runtime.hpp -- C++ host layer: the op-builder interface the reference's
// nn / Flux2 modules call (src/ggml/Runtime.hpp:7-317), method for method,
// over this library's ggml-shaped dt_tensor nodes instead of ggml_tensor.
//
// Nodes are recorded, not executed (the reference's Computation.hpp:13-22
// contract); HipRuntime::compute() plans fusion, allocates node memory with
// liveness reuse (ggml_gallocr's role) and runs the graph through
// dt_graph_compute, i.e. the C ABI in include/dit_hip.h.
#pragma once

#include <cstddef>
#include <cstdint>
#include <deque>
#include <memory>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "dit_hip.h"

namespace dit {
namespace host {

using Node = dt_tensor;

// ggml_op_pool / ggml_scale_mode stand-ins (ops this backend does not run).
enum class PoolOp { Max = 0, Avg = 1 };
enum class ScaleMode { Nearest = 0, Bilinear = 1 };

// Raised for Runtime methods outside this backend's op subset.
struct Unsupported : std::logic_error {
    using std::logic_error::logic_error;
};

// Raised when a C-ABI call fails (carries dt_last_error()).
struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void check(int rc, const char* what);

// Mirrors src/ggml/Runtime.hpp: same method names, argument order and meaning.
class Runtime {
public:
    virtual ~Runtime() = default;

    // Tensor creation / initialization (Runtime.hpp:15-41)
    virtual Node* new_tensor(int32_t type, int n_dims, const int64_t* ne) = 0;
    virtual Node* new_tensor_1d(int32_t type, int64_t ne0) = 0;
    virtual void set_input(Node* tensor) = 0;
    virtual void set_param(Node* tensor) = 0;
    virtual void set_output(Node* tensor) = 0;
    virtual Node* fill(Node* tensor, float value) = 0;

    // Copy / cast (:47-63)
    virtual Node* cont(Node* tensor) = 0;
    virtual Node* dup(Node* tensor) = 0;
    virtual Node* cast(Node* tensor, int32_t type) = 0;
    virtual Node* cpy(Node* src, Node* dst) = 0;

    // Unary arithmetic (:69-91)
    virtual Node* sqrt(Node* tensor) = 0;
    virtual Node* exp(Node* tensor) = 0;
    virtual Node* log(Node* tensor) = 0;
    virtual Node* sin(Node* tensor) = 0;
    virtual Node* cos(Node* tensor) = 0;
    virtual Node* sigmoid(Node* tensor) = 0;

    // Binary arithmetic: rhs broadcasts into lhs (:97-115)
    virtual Node* add(Node* lhs, Node* rhs) = 0;
    virtual Node* sub(Node* lhs, Node* rhs) = 0;
    virtual Node* mul(Node* lhs, Node* rhs) = 0;
    virtual Node* div(Node* lhs, Node* rhs) = 0;

    // Scalar arithmetic (:121-130)
    virtual Node* scale(Node* tensor, float value) = 0;
    virtual Node* clamp(Node* tensor, float min, float max) = 0;

    // Matrix operations (:136-139)
    virtual Node* mul_mat(Node* lhs, Node* rhs) = 0;

    // Reshape / permute / views (:145-221)
    virtual Node* reshape_1d(Node* tensor, int64_t ne0) = 0;
    virtual Node* reshape_2d(Node* tensor, int64_t ne0, int64_t ne1) = 0;
    virtual Node* reshape_3d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2) = 0;
    virtual Node* reshape_4d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) = 0;
    virtual Node* permute(Node* tensor, int axis0, int axis1, int axis2, int axis3) = 0;
    virtual Node* view_1d(Node* tensor, int64_t ne0, size_t offset) = 0;
    virtual Node* view_2d(Node* tensor, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) = 0;
    virtual Node* view_3d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1,
                          size_t nb2, size_t offset) = 0;
    virtual Node* view_4d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                          size_t nb1, size_t nb2, size_t nb3, size_t offset) = 0;

    // Repeat / concatenation / reduction (:227-248)
    virtual Node* repeat(Node* tensor, Node* target) = 0;
    virtual Node* concat(Node* a, Node* b, int dim) = 0;
    virtual Node* sum_rows(Node* tensor) = 0;

    // Attention, convolution, lookup (:250-271)
    virtual Node* flash_attn_ext(Node* q, Node* k, Node* v, Node* mask, float scale,
                                 float max_bias, float logit_softcap) = 0;
    virtual Node* conv_2d_direct(Node* a, Node* b, int s0, int s1, int p0, int p1, int d0,
                                 int d1) = 0;
    virtual Node* get_rows(Node* a, Node* b) = 0;

    // Norms and RoPE (:273-293)
    virtual Node* norm(Node* a, float eps) = 0;
    virtual Node* rms_norm(Node* a, float eps) = 0;
    virtual Node* rope_ext(Node* a, Node* b, Node* c, int n_dims, int mode, int n_ctx_orig,
                           float freq_base, float freq_scale, float ext_factor, float attn_factor,
                           float beta_fast, float beta_slow) = 0;

    // Pooling / resampling (:295-316)
    virtual Node* pool_2d(Node* a, PoolOp op, int k0, int k1, int s0, int s1, float p0,
                          float p1) = 0;
    virtual Node* interpolate(Node* a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                              uint32_t mode) = 0;
    virtual Node* upscale(Node* a, int scale_factor, ScaleMode mode) = 0;
};

// Statistics of the last HipRuntime::compute().
struct ComputeStats {
    int nodes = 0;
    int kernels = 0;
    int fused_nodes = 0;
    int mul_mat_nodes = 0;
    int attention_nodes = 0;
    int grouped_nodes = 0;      // run inside an earlier node's launch (grouped GEMMs)
    int deferred_nodes = 0;     // stored outputs computed by a later node's fused kernel
    size_t arena_bytes = 0;     // op-node memory after liveness reuse
    size_t naive_bytes = 0;     // the same nodes without reuse or fusion
    int launches_held = 0;      // fused launches the executor kept in node order (Allocation::NodeOrder)
    int fused_nodes_checked = 0;  // plan(): nodes fused after that check (Allocation::NodeOrder)
};

// The Runtime that records dt_tensor nodes and runs them on one HIP device.
// device < 0 makes a runtime without a device: graphs can be recorded and
// planned (plan()) but not computed.
class HipRuntime : public Runtime {
public:
    explicit HipRuntime(int device = 0, dt_stream_t stream = nullptr);
    ~HipRuntime() override;
    HipRuntime(const HipRuntime&) = delete;
    HipRuntime& operator=(const HipRuntime&) = delete;

    // ---- Runtime -----------------------------------------------------------
    Node* new_tensor(int32_t type, int n_dims, const int64_t* ne) override;
    Node* new_tensor_1d(int32_t type, int64_t ne0) override;
    void set_input(Node* tensor) override;
    void set_param(Node* tensor) override;
    void set_output(Node* tensor) override;
    Node* fill(Node* tensor, float value) override;
    Node* cont(Node* tensor) override;
    Node* dup(Node* tensor) override;
    Node* cast(Node* tensor, int32_t type) override;
    Node* cpy(Node* src, Node* dst) override;
    Node* sqrt(Node* tensor) override;
    Node* exp(Node* tensor) override;
    Node* log(Node* tensor) override;
    Node* sin(Node* tensor) override;
    Node* cos(Node* tensor) override;
    Node* sigmoid(Node* tensor) override;
    Node* add(Node* lhs, Node* rhs) override;
    Node* sub(Node* lhs, Node* rhs) override;
    Node* mul(Node* lhs, Node* rhs) override;
    Node* div(Node* lhs, Node* rhs) override;
    Node* scale(Node* tensor, float value) override;
    Node* clamp(Node* tensor, float min, float max) override;
    Node* mul_mat(Node* lhs, Node* rhs) override;
    Node* reshape_1d(Node* tensor, int64_t ne0) override;
    Node* reshape_2d(Node* tensor, int64_t ne0, int64_t ne1) override;
    Node* reshape_3d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2) override;
    Node* reshape_4d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) override;
    Node* permute(Node* tensor, int axis0, int axis1, int axis2, int axis3) override;
    Node* view_1d(Node* tensor, int64_t ne0, size_t offset) override;
    Node* view_2d(Node* tensor, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) override;
    Node* view_3d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1, size_t nb2,
                  size_t offset) override;
    Node* view_4d(Node* tensor, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1,
                  size_t nb2, size_t nb3, size_t offset) override;
    Node* repeat(Node* tensor, Node* target) override;
    Node* concat(Node* a, Node* b, int dim) override;
    Node* sum_rows(Node* tensor) override;
    Node* flash_attn_ext(Node* q, Node* k, Node* v, Node* mask, float scale, float max_bias,
                         float logit_softcap) override;
    Node* conv_2d_direct(Node* a, Node* b, int s0, int s1, int p0, int p1, int d0, int d1) override;
    Node* get_rows(Node* a, Node* b) override;
    Node* norm(Node* a, float eps) override;
    Node* rms_norm(Node* a, float eps) override;
    Node* rope_ext(Node* a, Node* b, Node* c, int n_dims, int mode, int n_ctx_orig, float freq_base,
                   float freq_scale, float ext_factor, float attn_factor, float beta_fast,
                   float beta_slow) override;
    Node* pool_2d(Node* a, PoolOp op, int k0, int k1, int s0, int s1, float p0, float p1) override;
    Node* interpolate(Node* a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                      uint32_t mode) override;
    Node* upscale(Node* a, int scale_factor, ScaleMode mode) override;

    // ---- data and execution ------------------------------------------------
    // Host bytes for a leaf (input or parameter), uploaded at every compute().
    void bind(Node* leaf, const void* host, size_t bytes);
    // Device memory the caller owns and keeps resident for a leaf (weights
    // loaded once, inputs already in HBM): never copied or freed here.
    void bind_device(Node* leaf, void* device_ptr);
    // Plan, allocate and run every recorded node; output nodes keep their data.
    // The plan and the device memory are kept while no node is added, so
    // repeated calls on the same graph only upload host-bound leaves and run.
    void compute();
    // compute(), replayed as one HIP graph (dt_graph_capture): the first call
    // after the plan changes runs eagerly and records the launches; later
    // calls upload host-bound leaves and submit the graph.  Same results.
    void compute_graph();
    // Fusion and memory plan of the recorded graph without touching a device;
    // fills stats() except `kernels`.
    const ComputeStats& plan();
    // Copy an output (or leaf) back to the host; `bytes` = its contiguous size.
    void read(const Node* node, void* host, size_t bytes) const;
    // Drop the recorded graph and its memory.
    void reset();

    // How node memory is placed.  Fused (the default): the arena follows the
    // fusion plan (absorbed nodes get no memory; outputs are placed where
    // their kernel runs, inputs kept until their last reader's kernel), so
    // the executor runs the plan as is (DT_GRAPH_ALLOC_RUNS_AT).  NodeOrder:
    // every op node gets memory at its own position, released after its last
    // reader in node order, in place over an input it is the last reader of
    // when the op allows -- ggml_gallocr's policy (Context.hpp:118-135); the
    // executor then checks its plan against those addresses.
    enum class Allocation { Fused, NodeOrder };
    void set_allocation(Allocation a);

    const ComputeStats& stats() const { return stats_; }
    dt_backend* backend() const { return be_; }
    // The recorded op and view nodes in creation (= execution) order.
    const std::vector<Node*>& nodes() const { return order_; }
    static size_t nbytes(const Node* t);

private:
    Node* make(int32_t type, const int64_t ne[4], int32_t op);
    Node* view_of(Node* src, const int64_t ne[4], const int64_t nb[4], size_t offset);
    Node* unary(Node* a, int32_t kind, float p0 = 0.f, float p1 = 0.f);
    Node* binary(int32_t op, Node* a, Node* b);
    Node* root_of(Node* t) const;

    dt_backend* be_ = nullptr;
    std::deque<Node> nodes_;                         // stable addresses
    std::vector<Node*> order_;                       // op and view nodes, creation order
    std::vector<Node*> leaves_;
    std::unordered_map<const Node*, std::vector<uint8_t>> host_data_;
    std::unordered_map<const Node*, void*> device_data_;
    bool prepared_ = false;
    void prepare(bool allocate = true);
    std::unordered_map<const Node*, Node*> alias_;   // cpy node -> destination
    void* leaf_buf_ = nullptr;
    void* arena_ = nullptr;
    size_t arena_cap_ = 0;
    ComputeStats stats_;
    dt_graph_exec* exec_ = nullptr;  // compute_graph's recording
    size_t plan_gen_ = 0, exec_gen_ = 0;  // prepare() count when it was recorded
    Allocation alloc_ = Allocation::Fused;
    uint32_t compute_flags() const { return alloc_ == Allocation::Fused ? (uint32_t)DT_GRAPH_ALLOC_RUNS_AT : 0u; }
    void upload_leaves();
    void resolve_alias_data();
};

// The runtime that module code uses (the reference's thread-local Scope,
// src/ggml/Scope.hpp:74-75).
Runtime& current_runtime();

class RuntimeScope {
public:
    explicit RuntimeScope(Runtime& rt);
    ~RuntimeScope();

private:
    Runtime* prev_;
};

}  // namespace host
}  // namespace dit
