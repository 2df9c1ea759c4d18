// tensor.hpp -- a PyTorch-shaped handle over a recorded node, with the
// reference Tensor's op-emission rules (src/ggml/Tensor.hpp, Tensor.cpp):
// shapes in PyTorch order (ggml ne[] reversed), binary operators that put
// the broadcast superset in ggml's src0 slot and lift both operands through
// an identity tensor when neither is a superset (Tensor.cpp:21-50, 97-190),
// scalars as filled one-element tensors (Tensor.hpp:229-236), views through
// narrow / chunk / select, reshape that first makes the source contiguous
// (Tensor.cpp:355-372) and pairwise left-nested cat (Tensor.cpp:252-299).
#pragma once

#include <cstdint>
#include <initializer_list>
#include <vector>

#include "runtime.hpp"

namespace dit {
namespace host {

class Tensor {
public:
    using Shape = std::vector<int64_t>;

    Tensor() = default;
    Tensor(Node* t, Shape shape);

    Node* operator*() const { return t_; }
    const Shape& shape() const { return shape_; }
    int64_t ndim() const { return (int64_t)shape_.size(); }
    int64_t size(int64_t dim) const;
    int64_t numel() const;
    int32_t dtype() const { return t_->type; }
    bool is_contiguous() const;

    // creation
    static Tensor empty(const Shape& shape, int32_t type);
    static Tensor full(const Shape& shape, float value, int32_t type = DT_TYPE_F32);
    static Tensor scalar(float value) { return full({}, value); }

    // arithmetic (operand order as the reference emits it)
    Tensor operator+(const Tensor& rhs) const;
    Tensor operator-(const Tensor& rhs) const;
    Tensor operator*(const Tensor& rhs) const;
    Tensor operator/(const Tensor& rhs) const;
    // Scalars as the reference's Tensor.hpp:351-369 takes them: + and - go
    // through a filled scalar tensor, * and / through ggml_scale.
    Tensor operator+(float rhs) const { return *this + scalar(rhs); }
    Tensor operator-(float rhs) const { return *this - scalar(rhs); }
    Tensor operator*(float rhs) const { return scale(rhs); }
    Tensor operator/(float rhs) const { return scale(1.0f / rhs); }
    Tensor operator-() const { return *this * -1.0f; }
    Tensor scale(float value) const;
    Tensor sigmoid() const;
    Tensor contiguous() const;

    // shape algebra
    Tensor reshape(Shape shape) const;
    Tensor narrow(int64_t dim, int64_t start, int64_t length) const;
    std::vector<Tensor> chunk(int n, int64_t dim) const;
    Tensor select(int64_t dim, int64_t index) const;  // x[..., index, ...]: narrow + squeeze
    Tensor squeeze(int64_t dim) const;
    Tensor unsqueeze(int64_t dim) const;
    Tensor unflatten(int64_t dim, const Shape& sizes) const;
    Tensor flatten(int64_t start_dim, int64_t end_dim) const;
    Tensor permute(const Shape& order) const;
    Tensor transpose(int64_t d0, int64_t d1) const;
    static Tensor cat(const std::vector<Tensor>& tensors, int64_t dim);

    static Shape broadcast(const Shape& a, const Shape& b);
    static int64_t normalize_dim(int64_t dim, int64_t rank, bool allow_end = false);

private:
    Node* t_ = nullptr;
    Shape shape_;
};

inline Tensor operator+(float v, const Tensor& t) { return t + v; }
inline Tensor operator*(float v, const Tensor& t) { return t * v; }
inline Tensor operator-(float v, const Tensor& t) { return Tensor::scalar(v) - t; }

}  // namespace host
}  // namespace dit
