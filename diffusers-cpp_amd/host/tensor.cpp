// tensor.cpp -- see tensor.hpp.  Every rule below restates how the
// reference's Tensor (src/ggml/Tensor.cpp) turns PyTorch-style expressions
// into Runtime calls; the node graph it records is what the executor's
// fusion pass pattern-matches, so operand order matters.
#include "tensor.hpp"

#include <stdexcept>

namespace dit {
namespace host {

namespace {

Runtime& rt() { return current_runtime(); }

// ggml ne of a PyTorch-order shape (rank 0 -> a 1-element vector).
void ggml_ne(const Tensor::Shape& s, int64_t ne[4]) {
    const int64_t r = (int64_t)s.size();
    for (int i = 0; i < 4; ++i) ne[i] = i < r ? s[r - 1 - i] : 1;
}

int64_t ggml_dim(const Tensor::Shape& s, int64_t i) {
    const int64_t r = (int64_t)s.size();
    return i < r ? s[r - 1 - i] : 1;
}

// Whether ggml can repeat b to a's shape: dim by dim (ggml order, absent
// dims taken as 1), b's extent has to divide a's, and an empty b never fits.
bool ggml_broadcasts(const Tensor::Shape& a, const Tensor::Shape& b) {
    const int64_t rank = (int64_t)std::max(a.size(), b.size());
    for (int64_t i = 0; i < rank; ++i) {
        const int64_t da = ggml_dim(a, i), db = ggml_dim(b, i);
        if (db == 0 || da % db != 0) return false;
    }
    return true;
}

Tensor identity(const Tensor::Shape& shape, int32_t type, float value) {
    Tensor blank = Tensor::empty(shape, type);
    return Tensor(rt().fill(*blank, value), shape);
}

bool node_contiguous(const Node* t) {
    int64_t expect = t->type == DT_TYPE_F32 || t->type == DT_TYPE_I32 ? 4 : 2;
    for (int i = 0; i < 4; ++i) {
        if (t->ne[i] > 1 && t->nb[i] != expect) return false;
        expect *= t->ne[i];
    }
    return true;
}

}  // namespace

Tensor::Tensor(Node* t, Shape shape) : t_(t), shape_(std::move(shape)) {
    if (shape_.size() > 4) throw std::invalid_argument("Tensor: at most 4 dims");
}

int64_t Tensor::normalize_dim(int64_t dim, int64_t rank, bool allow_end) {
    const int64_t upper = allow_end ? rank : rank - 1;
    if (dim < 0) dim += upper + 1;
    if (dim < 0 || dim > upper) throw std::out_of_range("dimension out of range");
    return dim;
}

int64_t Tensor::size(int64_t dim) const { return shape_[normalize_dim(dim, ndim())]; }

int64_t Tensor::numel() const {
    int64_t n = 1;
    for (int64_t d : shape_) n *= d;
    return n;
}

bool Tensor::is_contiguous() const { return node_contiguous(t_); }

Tensor Tensor::empty(const Shape& shape, int32_t type) {
    if (shape.empty()) return Tensor(rt().new_tensor_1d(type, 1), shape);
    int64_t ne[4];
    ggml_ne(shape, ne);
    return Tensor(rt().new_tensor(type, (int)shape.size(), ne), shape);
}

Tensor Tensor::full(const Shape& shape, float value, int32_t type) {
    return identity(shape, type, value);
}

Tensor::Shape Tensor::broadcast(const Shape& a, const Shape& b) {
    if (a.empty()) return b;
    if (b.empty()) return a;
    const size_t rank = std::max(a.size(), b.size());
    Shape out(rank);
    for (size_t i = 0; i < rank; ++i) {  // aligned from the last dim
        const int64_t da = i < a.size() ? a[a.size() - 1 - i] : 1;
        const int64_t db = i < b.size() ? b[b.size() - 1 - i] : 1;
        int64_t d;
        if (da == db || db == 1) d = da;
        else if (da == 1) d = db;
        else throw std::invalid_argument("shapes are not broadcastable");
        out[rank - 1 - i] = d;
    }
    return out;
}

// ---- binary operators (Tensor.cpp:97-190) ---------------------------------

Tensor Tensor::operator+(const Tensor& rhs) const {
    const Shape target = broadcast(shape_, rhs.shape_);
    if (ggml_broadcasts(shape_, rhs.shape_)) return Tensor(rt().add(t_, rhs.t_), target);
    if (ggml_broadcasts(rhs.shape_, shape_)) return Tensor(rt().add(rhs.t_, t_), target);
    Tensor lifted(rt().add(*identity(target, dtype(), 0.0f), t_), target);
    return Tensor(rt().add(lifted.t_, rhs.t_), target);
}

Tensor Tensor::operator-(const Tensor& rhs) const {
    const Shape target = broadcast(shape_, rhs.shape_);
    if (ggml_broadcasts(shape_, rhs.shape_)) return Tensor(rt().sub(t_, rhs.t_), target);
    if (ggml_broadcasts(rhs.shape_, shape_)) return -Tensor(rt().sub(rhs.t_, t_), target);
    Tensor lifted(rt().add(*identity(target, dtype(), 0.0f), t_), target);
    return Tensor(rt().sub(lifted.t_, rhs.t_), target);
}

Tensor Tensor::operator*(const Tensor& rhs) const {
    const Shape target = broadcast(shape_, rhs.shape_);
    if (ggml_broadcasts(shape_, rhs.shape_)) return Tensor(rt().mul(t_, rhs.t_), target);
    if (ggml_broadcasts(rhs.shape_, shape_)) return Tensor(rt().mul(rhs.t_, t_), target);
    Tensor lifted(rt().mul(*identity(target, dtype(), 1.0f), t_), target);
    return Tensor(rt().mul(lifted.t_, rhs.t_), target);
}

Tensor Tensor::operator/(const Tensor& rhs) const {
    const Shape target = broadcast(shape_, rhs.shape_);
    if (ggml_broadcasts(shape_, rhs.shape_)) return Tensor(rt().div(t_, rhs.t_), target);
    Tensor lifted(rt().add(*identity(target, dtype(), 0.0f), t_), target);
    return Tensor(rt().div(lifted.t_, rhs.t_), target);
}

Tensor Tensor::scale(float value) const { return Tensor(rt().scale(t_, value), shape_); }
Tensor Tensor::sigmoid() const { return Tensor(rt().sigmoid(t_), shape_); }
Tensor Tensor::contiguous() const { return Tensor(rt().cont(t_), shape_); }

// ---- shape algebra ---------------------------------------------------------

Tensor Tensor::reshape(Shape shape) const {
    int64_t known = 1, infer = -1;
    for (size_t i = 0; i < shape.size(); ++i) {
        if (shape[i] == -1) {
            if (infer >= 0) throw std::invalid_argument("reshape: only one -1 allowed");
            infer = (int64_t)i;
        } else {
            known *= shape[i];
        }
    }
    if (infer >= 0) {
        if (known == 0 || numel() % known) throw std::invalid_argument("reshape: incompatible shape");
        shape[infer] = numel() / known;
    } else if (known != numel()) {
        throw std::invalid_argument("reshape: incompatible shape");
    }
    Tensor src = is_contiguous() ? *this : contiguous();  // ggml_reshape needs contiguous input
    int64_t ne[4];
    ggml_ne(shape, ne);
    switch (shape.size()) {
        case 0: return Tensor(rt().reshape_1d(src.t_, 1), shape);
        case 1: return Tensor(rt().reshape_1d(src.t_, ne[0]), shape);
        case 2: return Tensor(rt().reshape_2d(src.t_, ne[0], ne[1]), shape);
        case 3: return Tensor(rt().reshape_3d(src.t_, ne[0], ne[1], ne[2]), shape);
        default: return Tensor(rt().reshape_4d(src.t_, ne[0], ne[1], ne[2], ne[3]), shape);
    }
}

Tensor Tensor::narrow(int64_t dim, int64_t start, int64_t length) const {
    const int64_t rank = ndim();
    dim = normalize_dim(dim, rank);
    const int64_t n = shape_[dim];
    if (start < 0) start += n;
    if (start < 0 || start > n || length < 0 || length > n - start)
        throw std::out_of_range("narrow: out of range");
    Shape out = shape_;
    out[dim] = length;
    const size_t offset = (size_t)start * (size_t)t_->nb[rank - 1 - dim];
    int64_t ne[4];
    ggml_ne(out, ne);
    switch (rank) {
        case 1: return Tensor(rt().view_1d(t_, ne[0], offset), out);
        case 2: return Tensor(rt().view_2d(t_, ne[0], ne[1], t_->nb[1], offset), out);
        case 3: return Tensor(rt().view_3d(t_, ne[0], ne[1], ne[2], t_->nb[1], t_->nb[2], offset), out);
        default:
            return Tensor(rt().view_4d(t_, ne[0], ne[1], ne[2], ne[3], t_->nb[1], t_->nb[2], t_->nb[3], offset),
                          out);
    }
}

std::vector<Tensor> Tensor::chunk(int n, int64_t dim) const {
    if (n <= 0) throw std::invalid_argument("chunk: n must be positive");
    dim = normalize_dim(dim, ndim());
    const int64_t total = shape_[dim], split = (total + n - 1) / n;
    std::vector<Tensor> out;
    for (int64_t s = 0; s < total; s += split) out.push_back(narrow(dim, s, std::min(split, total - s)));
    return out;
}

Tensor Tensor::squeeze(int64_t dim) const {
    dim = normalize_dim(dim, ndim());
    if (shape_[dim] != 1) throw std::invalid_argument("squeeze: dimension is not 1");
    Shape out;
    for (int64_t i = 0; i < ndim(); ++i)
        if (i != dim) out.push_back(shape_[i]);
    return reshape(out);
}

Tensor Tensor::select(int64_t dim, int64_t index) const {
    dim = normalize_dim(dim, ndim());
    if (index < 0) index += shape_[dim];
    return narrow(dim, index, 1).squeeze(dim);
}

Tensor Tensor::unsqueeze(int64_t dim) const {
    dim = normalize_dim(dim, ndim(), true);
    Shape out = shape_;
    out.insert(out.begin() + dim, 1);
    return reshape(out);
}

Tensor Tensor::unflatten(int64_t dim, const Shape& sizes) const {
    dim = normalize_dim(dim, ndim());
    Shape out(shape_.begin(), shape_.begin() + dim);
    out.insert(out.end(), sizes.begin(), sizes.end());
    out.insert(out.end(), shape_.begin() + dim + 1, shape_.end());
    return reshape(out);
}

Tensor Tensor::flatten(int64_t start_dim, int64_t end_dim) const {
    start_dim = normalize_dim(start_dim, ndim());
    end_dim = normalize_dim(end_dim, ndim());
    if (start_dim > end_dim) throw std::invalid_argument("flatten: start > end");
    Shape out(shape_.begin(), shape_.begin() + start_dim);
    int64_t m = 1;
    for (int64_t i = start_dim; i <= end_dim; ++i) m *= shape_[i];
    out.push_back(m);
    out.insert(out.end(), shape_.begin() + end_dim + 1, shape_.end());
    return reshape(out);
}

Tensor Tensor::permute(const Shape& order) const {
    const int64_t rank = ndim();
    if ((int64_t)order.size() != rank) throw std::invalid_argument("permute: order rank mismatch");
    // Output PyTorch dim i takes input dim order[i]; in ggml axes the input
    // axis (rank-1-order[i]) moves to output axis (rank-1-i).
    int ax[4] = {0, 1, 2, 3};
    Shape out(rank);
    for (int64_t i = 0; i < rank; ++i) {
        const int64_t src = normalize_dim(order[i], rank);
        ax[rank - 1 - src] = (int)(rank - 1 - i);
        out[i] = shape_[src];
    }
    return Tensor(rt().permute(t_, ax[0], ax[1], ax[2], ax[3]), out);
}

Tensor Tensor::transpose(int64_t d0, int64_t d1) const {
    Shape order(ndim());
    for (int64_t i = 0; i < ndim(); ++i) order[i] = i;
    std::swap(order[normalize_dim(d0, ndim())], order[normalize_dim(d1, ndim())]);
    return permute(order);
}

Tensor Tensor::cat(const std::vector<Tensor>& tensors, int64_t dim) {
    if (tensors.empty()) throw std::invalid_argument("cat: empty list");
    const Tensor& first = tensors.front();
    const int64_t rank = first.ndim();
    dim = normalize_dim(dim, rank);
    Shape out = first.shape();
    out[dim] = 0;
    for (const Tensor& t : tensors) {
        if (t.ndim() != rank || t.dtype() != first.dtype())
            throw std::invalid_argument("cat: rank or dtype mismatch");
        for (int64_t d = 0; d < rank; ++d)
            if (d != dim && t.shape()[d] != first.shape()[d])
                throw std::invalid_argument("cat: sizes differ outside the cat dimension");
        out[dim] += t.shape()[dim];
    }
    Node* acc = *first;
    for (size_t i = 1; i < tensors.size(); ++i)
        acc = rt().concat(acc, *tensors[i], (int)(rank - 1 - dim));
    return Tensor(acc, out);
}

}  // namespace host
}  // namespace dit
