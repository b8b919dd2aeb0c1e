// irontensor.hpp -- C++ host API of the MI355X matmul path, header-only over the C ABI
// (irontensor_hip.h). It mirrors IronTensor's Rust API for this path: the same names, argument
// meaning and error behaviour, so code written against the reference's Tensor/ops reads the same.
//
//   Rust                                  here
//   TensorResult<Tensor> / TensorError    returns Tensor, throws irontensor::TensorError subclasses
//   panic!/assert!/expect                 throws irontensor::Panic
//   MetalContext::global()                irontensor::Context::global()
//   CommandBatch::{begin,sync,...}        irontensor::CommandBatch (same static names)
//
// Tensors own device memory from the library's caching allocator; host reads synchronise the
// stream and copy out (the reference reads unified memory after a sync, src/tensor.rs:136-159).
#pragma once

#include <cmath>
#include <cstdint>
#include <cstring>
#include <memory>
#include <limits>
#include <numeric>
#include <sstream>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "irontensor_hip.h"

namespace irontensor {

// ------------------------------------------------------------------ errors (src/error.rs:7-71)

inline std::string shape_str(const std::vector<size_t> &s) {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < s.size(); ++i) o << (i ? ", " : "") << s[i];
    o << "]";
    return o.str();
}

struct TensorError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct ShapeMismatch : TensorError {
    ShapeMismatch(const std::string &op, const std::string &expected, const std::string &got)
        : TensorError(op + ": shape mismatch, expected " + expected + ", got " + got) {}
};
struct UnsupportedDimensions : TensorError {
    UnsupportedDimensions(const std::string &op, const std::string &expected, const std::vector<size_t> &got)
        : TensorError(op + ": unsupported dimensions, expected " + expected + ", got " + shape_str(got)) {}
};
struct PrecisionMismatch : TensorError {
    PrecisionMismatch(const std::string &op, const std::string &expected, const std::string &got)
        : TensorError(op + ": precision mismatch, expected " + expected + ", got " + got) {}
};
struct InnerDimensionMismatch : TensorError {
    InnerDimensionMismatch(const std::string &op, const std::vector<size_t> &a, const std::vector<size_t> &b)
        : TensorError(op + ": inner dimensions don't match, A=" + shape_str(a) + ", B=" + shape_str(b)) {}
};
struct EmptyTensor : TensorError {
    explicit EmptyTensor(const std::string &op) : TensorError(op + ": empty tensor not supported") {}
};
struct InvalidValue : TensorError {
    InvalidValue(const std::string &op, const std::string &msg) : TensorError(op + ": " + msg) {}
};
// Where the reference panics (assert!, assert_eq!, expect).
struct Panic : std::logic_error {
    using std::logic_error::logic_error;
};
// HIP runtime failures, allocation failure, missing device (the reference panics on these).
struct DeviceError : std::runtime_error {
    it_status status;
    DeviceError(it_status st, const std::string &m) : std::runtime_error(m), status(st) {}
};

inline void check(it_status st, const char *op) {
    if (st == IT_OK) return;
    std::string msg = it_last_error();
    switch (st) {
    case IT_ERR_PRECISION: throw TensorError(msg);
    case IT_ERR_INVALID:
    case IT_ERR_NULL:
    case IT_ERR_SHAPE:
    case IT_ERR_DIMS:
    case IT_ERR_INNER_DIM: throw InvalidValue(op, msg);
    default: throw DeviceError(st, std::string("[") + it_status_string(st) + "] " + msg);
    }
}

// ------------------------------------------------------------------ precision (src/precision.rs)

enum class Precision : int { FP32 = IT_F32, FP16 = IT_F16, BF16 = IT_BF16 };

inline size_t byte_size(Precision p) { return p == Precision::FP32 ? 4 : 2; }
inline const char *precision_name(Precision p) {
    return p == Precision::FP32 ? "FP32" : p == Precision::BF16 ? "BF16" : "unknown";
}

// src/precision.rs:24-29 (round to nearest even by adding 0x7FFF + lsb; NaN payload quirk kept).
inline uint16_t f32_to_bf16(float x) {
    uint32_t bits;
    std::memcpy(&bits, &x, 4);
    const uint32_t round = ((bits >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((bits + round) >> 16);
}
// src/precision.rs:33-35
inline float bf16_to_f32(uint16_t x) {
    const uint32_t bits = (uint32_t)x << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// ------------------------------------------------------------------ context (src/device.rs)

class Context {
  public:
    static Context &global() {
        static Context ctx(0);
        return ctx;
    }
    explicit Context(int device) { check(it_init(device, &handle_), "it_init"); }
    ~Context() {
        if (handle_) it_shutdown(handle_);
    }
    Context(const Context &) = delete;
    Context &operator=(const Context &) = delete;
    it_context *handle() const { return handle_; }
    void sync() const { check(it_stream_sync(handle_), "sync"); }
    size_t current_allocated_size() const { return it_mem_allocated(handle_); }

  private:
    it_context *handle_ = nullptr;
};

// gpu_memory_allocated (src/device.rs:43-71)
inline size_t gpu_memory_allocated() { return Context::global().current_allocated_size(); }

// ------------------------------------------------------------------ Tensor (src/tensor.rs)

class Tensor {
    struct Buffer {
        it_context *ctx;
        void *ptr = nullptr;
        Buffer(it_context *c, size_t bytes) : ctx(c) {
            check(it_malloc(ctx, bytes ? bytes : 1, &ptr), "alloc");
        }
        ~Buffer() { it_free(ctx, ptr); }
    };

  public:
    static size_t numel_of(const std::vector<size_t> &s) {
        return std::accumulate(s.begin(), s.end(), (size_t)1, std::multiplies<size_t>());
    }
    // Uninitialised tensor for outputs a kernel fully overwrites.
    static Tensor empty(const std::vector<size_t> &shape, Precision p) {
        return Tensor(std::make_shared<Buffer>(Context::global().handle(), numel_of(shape) * irontensor::byte_size(p)), shape, p);
    }
    static Tensor zeros(const std::vector<size_t> &shape, Precision p) {
        Tensor t = empty(shape, p);
        if (t.byte_size()) check(it_zero(Context::global().handle(), t.data(), t.byte_size()), "zeros");
        return t;
    }
    static Tensor from_f32_slice(const std::vector<float> &data, const std::vector<size_t> &shape) {
        return upload(data.data(), data.size(), shape, Precision::FP32);
    }
    static Tensor from_bf16_slice(const std::vector<uint16_t> &data, const std::vector<size_t> &shape) {
        return upload(data.data(), data.size(), shape, Precision::BF16);
    }
    static Tensor from_f32_as_bf16(const std::vector<float> &data, const std::vector<size_t> &shape) {
        std::vector<uint16_t> h(data.size());
        for (size_t i = 0; i < data.size(); ++i) h[i] = f32_to_bf16(data[i]);
        return from_bf16_slice(h, shape);
    }

    const std::vector<size_t> &shape() const { return shape_; }
    Precision precision() const { return prec_; }
    size_t numel() const { return numel_of(shape_); }
    size_t byte_size() const { return numel() * irontensor::byte_size(prec_); }
    bool is_f32() const { return prec_ == Precision::FP32; }
    bool is_bf16() const { return prec_ == Precision::BF16; }
    void *data() const { return buf_->ptr; }

    std::vector<float> as_f32_slice() const {
        if (prec_ != Precision::FP32) throw Panic("Tensor precision is not FP32");
        std::vector<float> out(numel());
        download(out.data(), out.size() * 4);
        return out;
    }
    std::vector<uint16_t> as_bf16_slice() const {
        if (prec_ != Precision::BF16) throw Panic("Tensor precision is not BF16");
        std::vector<uint16_t> out(numel());
        download(out.data(), out.size() * 2);
        return out;
    }
    Tensor view(const std::vector<size_t> &new_shape) const {
        if (numel_of(new_shape) != numel())
            throw Panic("Cannot view tensor of " + std::to_string(numel()) + " elements as shape " + shape_str(new_shape));
        return Tensor(buf_, new_shape, prec_);
    }
    void reshape(const std::vector<size_t> &new_shape) {
        if (numel_of(new_shape) != numel())
            throw Panic("Cannot reshape tensor of " + std::to_string(numel()) + " elements to shape " + shape_str(new_shape));
        shape_ = new_shape;
    }
    Tensor clone() const {
        Tensor t = empty(shape_, prec_);
        if (byte_size()) check(it_memcpy_d2d(Context::global().handle(), t.data(), data(), byte_size()), "clone");
        return t;
    }
    Tensor to_bf16() const {
        if (prec_ != Precision::FP32) throw Panic("to_bf16() requires FP32 tensor");
        std::vector<float> f = as_f32_slice();
        return from_f32_as_bf16(f, shape_);
    }
    Tensor to_f32() const {
        if (prec_ != Precision::BF16) throw Panic("to_f32() requires BF16 tensor");
        std::vector<uint16_t> h = as_bf16_slice();
        std::vector<float> f(h.size());
        for (size_t i = 0; i < h.size(); ++i) f[i] = bf16_to_f32(h[i]);
        return from_f32_slice(f, shape_);
    }

  private:
    Tensor(std::shared_ptr<Buffer> b, std::vector<size_t> s, Precision p) : buf_(std::move(b)), shape_(std::move(s)), prec_(p) {}
    static Tensor upload(const void *src, size_t n, const std::vector<size_t> &shape, Precision p) {
        if (n != numel_of(shape))
            throw Panic("Data length " + std::to_string(n) + " does not match shape " + shape_str(shape) +
                        " (numel=" + std::to_string(numel_of(shape)) + ")");
        Tensor t = empty(shape, p);
        if (n) check(it_memcpy_h2d(Context::global().handle(), t.data(), src, t.byte_size()), "upload");
        return t;
    }
    void download(void *dst, size_t bytes) const {
        if (bytes) check(it_memcpy_d2h(Context::global().handle(), dst, data(), bytes), "download");
    }

    std::shared_ptr<Buffer> buf_;
    std::vector<size_t> shape_;
    Precision prec_;
};

// ------------------------------------------------------------------ CommandBatch (src/command_batch.rs)
// Work is always stream-ordered on the context's single stream; begin() is a no-op, sync() waits,
// and commit_async()/wait_for_completion() use an event, as the reference's modes do.
class CommandBatch {
  public:
    static void begin() { active() = true; }
    static bool is_active() { return active(); }
    static void sync() { Context::global().sync(); }
    static void end() {
        sync();
        active() = false;
    }
    static void commit_async() {
        it_event *&ev = pending();
        if (!ev) check(it_event_create(Context::global().handle(), &ev), "commit_async");
        check(it_event_record(Context::global().handle(), ev), "commit_async");
    }
    static bool is_async_complete() {
        it_event *ev = pending();
        if (!ev) return true;
        it_status st = it_event_query(ev);
        if (st == IT_ERR_NOT_READY) return false;
        check(st, "is_async_complete");
        return true;
    }
    static void wait_for_completion() {
        if (it_event *ev = pending()) check(it_event_sync(ev), "wait_for_completion");
    }

  private:
    static bool &active() {
        static thread_local bool a = false;
        return a;
    }
    static it_event *&pending() {
        static thread_local it_event *e = nullptr;
        return e;
    }
};

// ------------------------------------------------------------------ ops

namespace detail {
inline Tensor gemm(const Tensor &a, const Tensor &b, bool ta, bool tb, const char *op,
                   Precision out_prec = Precision::FP32, const Tensor *bias = nullptr, float alpha = 1.f) {
    const auto &sa = a.shape(), &sb = b.shape();
    const bool batched = sa.size() == 3;
    const size_t batch = batched ? sa[0] : 1;
    const size_t ra = sa[sa.size() - 2], ca = sa[sa.size() - 1];
    const size_t rb = sb[sb.size() - 2], cb = sb[sb.size() - 1];
    const size_t M = ta ? ca : ra, K = ta ? ra : ca, N = tb ? rb : cb;
    Tensor c = Tensor::empty(batched ? std::vector<size_t>{batch, M, N} : std::vector<size_t>{M, N}, out_prec);
    it_epilogue epi{};
    if (bias) {
        epi.flags = IT_EPI_BIAS;
        epi.bias = (const float *)bias->data();
    }
    check(it_gemm(Context::global().handle(), (it_dtype)a.precision(), (it_dtype)out_prec, ta ? IT_OP_T : IT_OP_N,
                  tb ? IT_OP_T : IT_OP_N, (int64_t)M, (int64_t)N, (int64_t)K, alpha, a.data(), (int64_t)ca,
                  batched ? (int64_t)(ra * ca) : 0, b.data(), (int64_t)cb, sb.size() == 3 ? (int64_t)(rb * cb) : 0,
                  0.f, c.data(), (int64_t)N, batched ? (int64_t)(M * N) : 0, (int64_t)batch, bias ? &epi : nullptr),
          op);
    return c;
}

inline void require(bool cond, const std::string &msg) {
    if (!cond) throw Panic(msg);
}
}  // namespace detail

// src/ops/mps_gemm.rs:44-91 -- C = A.B, FP32, 2D or 3D; TensorError on precision/rank/inner/batch.
inline Tensor matmul_mps(const Tensor &a, const Tensor &b) {
    for (const Tensor *t : {&a, &b})
        if (t->precision() != Precision::FP32)
            throw PrecisionMismatch("matmul", "FP32", t->precision() == Precision::BF16 ? "BF16" : "unknown");
    const auto &sa = a.shape(), &sb = b.shape();
    if (sa.size() == 2 && sb.size() == 2) {
        if (sa[1] != sb[0]) throw InnerDimensionMismatch("matmul", sa, sb);
        return detail::gemm(a, b, false, false, "matmul");
    }
    if (sa.size() == 3 && sb.size() == 3) {
        if (sa[0] != sb[0])
            throw ShapeMismatch("matmul_batched", "batch size " + std::to_string(sa[0]), "batch size " + std::to_string(sb[0]));
        if (sa[2] != sb[1]) throw InnerDimensionMismatch("matmul_batched", sa, sb);
        return detail::gemm(a, b, false, false, "matmul_batched");
    }
    throw UnsupportedDimensions("matmul", "2D or 3D tensors", {sa.size(), sb.size()});
}

// src/ops/gemm.rs:88-91
inline Tensor matmul(const Tensor &a, const Tensor &b) { return matmul_mps(a, b); }

// src/ops/gemm.rs:102-285 -- same contract, panicking.
inline Tensor matmul_custom(const Tensor &a, const Tensor &b) {
    try {
        return matmul_mps(a, b);
    } catch (const TensorError &e) {
        throw Panic(e.what());
    }
}

// src/ops/mps_gemm.rs:213-314 -- Y = A.B^T, A [M,K], B [N,K].
inline Tensor matmul_mps_nt(const Tensor &a, const Tensor &b) {
    detail::require(a.is_f32() && b.is_f32(), "MPS matmul currently only supports FP32");
    detail::require(a.shape().size() == 2 && b.shape().size() == 2, "matmul_mps_nt requires 2D tensors");
    const auto &sa = a.shape(), &sb = b.shape();
    detail::require(sa[1] == sb[1], "Inner dimensions must match: A[" + std::to_string(sa[0]) + ", " +
                                        std::to_string(sa[1]) + "] @ B[" + std::to_string(sb[0]) + ", " +
                                        std::to_string(sb[1]) + "]^T");
    return detail::gemm(a, b, false, true, "matmul_mps_nt");
}

// src/ops/mps_gemm.rs:325-426 -- C = A^T.B, A [K,M], B [K,N].
inline Tensor matmul_mps_tn(const Tensor &a, const Tensor &b) {
    detail::require(a.is_f32() && b.is_f32(), "MPS matmul currently only supports FP32");
    detail::require(a.shape().size() == 2 && b.shape().size() == 2, "matmul_mps_tn requires 2D tensors");
    const auto &sa = a.shape(), &sb = b.shape();
    detail::require(sa[0] == sb[0], "Inner dimensions must match: A[" + std::to_string(sa[0]) + ", " +
                                        std::to_string(sa[1]) + "]^T @ B[" + std::to_string(sb[0]) + ", " +
                                        std::to_string(sb[1]) + "]");
    return detail::gemm(a, b, true, false, "matmul_mps_tn");
}

// src/train/helpers.rs:80-83
inline Tensor matmul_tn(const Tensor &a, const Tensor &b) { return matmul_mps_tn(a, b); }

// src/ops/backward/gemm.rs:106-133 -- grad_A = grad_C . B^T
inline Tensor matmul_backward_a(const Tensor &grad_c, const Tensor &b) {
    detail::require(grad_c.is_f32() && b.is_f32(), "matmul_backward_a requires FP32");
    const auto &g = grad_c.shape(), &s = b.shape();
    if (g.size() == 2 && s.size() == 2)
        detail::require(s[1] == g[1], "assertion `left == right` failed");
    else if (g.size() == 3 && s.size() == 3)
        detail::require(s[0] == g[0] && s[2] == g[2], "assertion `left == right` failed");
    else
        throw Panic("Unsupported shapes for matmul_backward_a");
    return detail::gemm(grad_c, b, false, true, "matmul_backward_a");
}

// src/ops/backward/gemm.rs:136-163 -- grad_B = A^T . grad_C
inline Tensor matmul_backward_b(const Tensor &grad_c, const Tensor &a) {
    detail::require(grad_c.is_f32() && a.is_f32(), "matmul_backward_b requires FP32");
    const auto &g = grad_c.shape(), &s = a.shape();
    if (g.size() == 2 && s.size() == 2)
        detail::require(s[0] == g[0], "assertion `left == right` failed");
    else if (g.size() == 3 && s.size() == 3)
        detail::require(s[0] == g[0] && s[1] == g[1], "assertion `left == right` failed");
    else
        throw Panic("Unsupported shapes for matmul_backward_b");
    return detail::gemm(a, grad_c, true, false, "matmul_backward_b");
}

// src/ops/backward/gemm.rs:73-103 -- 2D, 3D, or 4D (leading dims collapsed).
inline std::pair<Tensor, Tensor> matmul_backward(const Tensor &grad_c, const Tensor &a, const Tensor &b) {
    const auto &sa = a.shape(), &sb = b.shape();
    if (sa.size() == 4 && sb.size() == 4) {
        const size_t bt = sa[0] * sa[1];
        const auto &sg = grad_c.shape();
        auto r = matmul_backward(grad_c.view({bt, sg[2], sg[3]}), a.view({bt, sa[2], sa[3]}), b.view({bt, sb[2], sb[3]}));
        return {r.first.view(sa), r.second.view(sb)};
    }
    if (!((sa.size() == 2 && sb.size() == 2) || (sa.size() == 3 && sb.size() == 3)))
        throw Panic("matmul_backward requires 2D, 3D, or 4D tensors, got shapes " + shape_str(sa) + " and " + shape_str(sb));
    return {matmul_backward_a(grad_c, b), matmul_backward_b(grad_c, a)};
}

// src/ops/bf16_ops/precision.rs:15-78
inline Tensor to_bf16_gpu(const Tensor &t) {
    if (t.is_bf16()) return t.clone();
    Tensor out = Tensor::empty(t.shape(), Precision::BF16);
    check(it_f32_to_bf16(Context::global().handle(), (const float *)t.data(), (uint16_t *)out.data(), (int64_t)t.numel()), "to_bf16_gpu");
    return out;
}
inline Tensor to_f32_gpu(const Tensor &t) {
    if (t.is_f32()) return t.clone();
    Tensor out = Tensor::empty(t.shape(), Precision::FP32);
    check(it_bf16_to_f32(Context::global().handle(), (const uint16_t *)t.data(), (float *)out.data(), (int64_t)t.numel()), "to_f32_gpu");
    return out;
}

// src/ops/bf16_ops/gemm.rs:25-82 and :85-146 -- BF16 in, FP32 accumulate, BF16 out.
inline Tensor matmul_bf16(const Tensor &a, const Tensor &b) {
    detail::require(a.is_bf16(), "matmul_bf16 requires BF16 input A");
    detail::require(b.is_bf16(), "matmul_bf16 requires BF16 input B");
    detail::require(a.shape().size() == 2 && b.shape().size() == 2, "matmul_bf16 requires 2D tensors");
    detail::require(a.shape()[1] == b.shape()[0], "Inner dimensions must match");
    return detail::gemm(a, b, false, false, "matmul_bf16", Precision::BF16);
}
inline Tensor matmul_bf16_batched(const Tensor &a, const Tensor &b) {
    detail::require(a.is_bf16() && b.is_bf16(), "assertion `left == right` failed");
    detail::require(a.shape().size() == 3 && b.shape().size() == 3, "batched matmul requires 3D tensors");
    detail::require(a.shape()[0] == b.shape()[0], "Batch dimensions must match");
    detail::require(a.shape()[2] == b.shape()[1], "Inner dimensions must match");
    return detail::gemm(a, b, false, false, "matmul_bf16_batched", Precision::BF16);
}

// src/train/helpers.rs:12-18, :48-53, :61-76
inline Tensor ensure_fp32(const Tensor &t) { return t.is_bf16() ? to_f32_gpu(t) : t; }
inline Tensor linear_forward(const Tensor &input, const Tensor &weight) {
    return matmul_mps_nt(input, ensure_fp32(weight));
}
inline std::pair<Tensor, Tensor> linear_backward(const Tensor &grad_output, const Tensor &input, const Tensor &weight) {
    Tensor w = ensure_fp32(weight);
    return {matmul(grad_output, w), matmul_tn(grad_output, input)};
}

// nn::Linear::forward (src/nn/linear.rs:87-145) with the bias fused into the GEMM epilogue.
inline Tensor linear(const Tensor &input, const Tensor &weight, const Tensor *bias = nullptr) {
    const auto &s = input.shape();
    detail::require(!s.empty(), "Input must have at least one dimension");
    const size_t out_f = weight.shape()[0], in_f = weight.shape()[1];
    detail::require(s.back() == in_f, "Input last dimension " + std::to_string(s.back()) +
                                          " doesn't match in_features " + std::to_string(in_f));
    size_t rows = 1;
    for (size_t i = 0; i + 1 < s.size(); ++i) rows *= s[i];
    Tensor x = ensure_fp32(input), w = ensure_fp32(weight);
    Tensor y = bias ? [&] {
        Tensor bb = ensure_fp32(*bias);
        return detail::gemm(x.view({rows, in_f}), w, false, true, "linear", Precision::FP32, &bb);
    }()
                    : detail::gemm(x.view({rows, in_f}), w, false, true, "linear");
    if (s.size() > 2) {
        std::vector<size_t> os(s.begin(), s.end() - 1);
        os.push_back(out_f);
        return y.view(os);
    }
    return y;
}

// ops::attention (src/ops/attention.rs:286-377): [B,S,H,D] FP32, addressed in place per head.
inline Tensor attention(const Tensor &q, const Tensor &k, const Tensor &v, bool causal) {
    detail::require(q.is_f32() && k.is_f32() && v.is_f32(), "assertion `left == right` failed: attention requires FP32");
    detail::require(q.shape().size() == 4, "Q must be 4D [batch, seq, heads, dim]");
    detail::require(k.shape().size() == 4, "K must be 4D [batch, seq, heads, dim]");
    detail::require(v.shape().size() == 4, "V must be 4D [batch, seq, heads, dim]");
    const size_t b = q.shape()[0], sq = q.shape()[1], h = q.shape()[2], d = q.shape()[3], skv = k.shape()[1];
    detail::require(k.shape()[0] == b && v.shape()[0] == b, "Batch size mismatch");
    detail::require(k.shape()[2] == h && v.shape()[2] == h, "Num heads mismatch");
    detail::require(k.shape()[3] == d && v.shape()[3] == d, "Head dim mismatch");
    detail::require(v.shape()[1] == skv, "K and V seq_len must match");
    if (b == 0 || sq == 0 || skv == 0) return Tensor::zeros({b, sq, h, d}, Precision::FP32);
    detail::require(!causal || sq == skv, "Causal attention requires Q and K to have same seq_len");
    Tensor out = Tensor::empty({b, sq, h, d}, Precision::FP32);
    Tensor sc = Tensor::empty({b * h, sq, skv}, Precision::FP32);
    Tensor p = Tensor::empty({b * h, sq, skv}, Precision::FP32);
    it_attn_layout lq{(int64_t)h, (int64_t)(sq * h * d), (int64_t)d, (int64_t)(h * d)};
    it_attn_layout lkv{(int64_t)h, (int64_t)(skv * h * d), (int64_t)d, (int64_t)(h * d)};
    check(it_attention_forward(Context::global().handle(), IT_F32, (int64_t)(b * h), (int64_t)sq, (int64_t)skv,
                               (int64_t)d, 1.f / std::sqrt((float)d), causal ? 1 : 0, &lq, &lkv, &lq, q.data(),
                               k.data(), v.data(), (float *)sc.data(), p.data(), (float *)out.data()),
          "attention");
    return out;
}

// ops::attention on [B,S,H,D], fused for head_dim 64 (no [seq, seq] buffers; other head_dim up to
// 128 run the materialised contractions); same checks as attention().
inline Tensor flash_attention_bshd(const Tensor &q, const Tensor &k, const Tensor &v, bool causal) {
    detail::require(q.is_f32() && k.is_f32() && v.is_f32(), "assertion `left == right` failed: attention requires FP32");
    detail::require(q.shape().size() == 4, "Q must be 4D [batch, seq, heads, dim]");
    detail::require(k.shape().size() == 4, "K must be 4D [batch, seq, heads, dim]");
    detail::require(v.shape().size() == 4, "V must be 4D [batch, seq, heads, dim]");
    const size_t b = q.shape()[0], sq = q.shape()[1], h = q.shape()[2], d = q.shape()[3], skv = k.shape()[1];
    detail::require(k.shape()[0] == b && v.shape()[0] == b, "Batch size mismatch");
    detail::require(k.shape()[2] == h && v.shape()[2] == h, "Num heads mismatch");
    detail::require(k.shape()[3] == d && v.shape()[3] == d, "Head dim mismatch");
    detail::require(v.shape()[1] == skv, "K and V seq_len must match");
    if (b == 0 || sq == 0 || skv == 0) return Tensor::zeros({b, sq, h, d}, Precision::FP32);
    detail::require(!causal || sq == skv, "Causal attention requires Q and K to have same seq_len");
    Tensor out = Tensor::empty({b, sq, h, d}, Precision::FP32);
    it_attn_layout lq{(int64_t)h, (int64_t)(sq * h * d), (int64_t)d, (int64_t)(h * d)};
    it_attn_layout lkv{(int64_t)h, (int64_t)(skv * h * d), (int64_t)d, (int64_t)(h * d)};
    check(it_flash_attention_forward(Context::global().handle(), IT_F32, (int64_t)(b * h), (int64_t)sq,
                                     (int64_t)skv, (int64_t)d, 1.f / std::sqrt((float)d), causal ? 1 : 0, &lq,
                                     &lkv, &lq, q.data(), k.data(), v.data(), (float *)out.data(), nullptr),
          "attention");
    return out;
}

// flash_attention (src/ops/flash_attention.rs:76-193, re-exported at src/ops/mod.rs:36): attention
// on [batch, heads, seq, head_dim] FP32 tensors of one shape, scale 1/sqrt(head_dim), head_dim <= 128;
// same assertions and messages; zeros at seq 0. head_dim 64 runs the fused kernels, other sizes the
// materialised contractions.
inline Tensor flash_attention(const Tensor &q, const Tensor &k, const Tensor &v, bool causal) {
    detail::require(q.is_f32(), "assertion `left == right` failed: Q must be FP32");
    detail::require(k.is_f32(), "assertion `left == right` failed: K must be FP32");
    detail::require(v.is_f32(), "assertion `left == right` failed: V must be FP32");
    detail::require(q.shape().size() == 4, "Q must be 4D [batch, heads, seq, head_dim]");
    detail::require(k.shape().size() == 4, "K must be 4D [batch, heads, seq, head_dim]");
    detail::require(v.shape().size() == 4, "V must be 4D [batch, heads, seq, head_dim]");
    detail::require(q.shape() == k.shape(), "Q and K must have same shape");
    detail::require(q.shape() == v.shape(), "Q and V must have same shape");
    const size_t b = q.shape()[0], h = q.shape()[1], s = q.shape()[2], d = q.shape()[3];
    detail::require(d <= 128, "head_dim must be <= 128");
    if (b * h * s * d == 0) return Tensor::zeros({b, h, s, d}, Precision::FP32);
    Tensor out = Tensor::empty({b, h, s, d}, Precision::FP32);
    check(it_flash_attention_forward(Context::global().handle(), IT_F32, (int64_t)(b * h), (int64_t)s, (int64_t)s,
                                     (int64_t)d, 1.f / std::sqrt((float)d), causal ? 1 : 0, nullptr, nullptr,
                                     nullptr, q.data(), k.data(), v.data(), (float *)out.data(), nullptr),
          "flash_attention");
    return out;
}

// attention_backward_recompute (src/train/helpers.rs:120-193) on [B,H,S,D]: (dQ, dK, dV).
struct AttentionGrads {
    Tensor dq, dk, dv;
};
inline AttentionGrads attention_backward_recompute(const Tensor &grad_output, const Tensor &q, const Tensor &k,
                                                    const Tensor &v) {
    const auto &s = q.shape();
    detail::require(s.size() == 4, "attention_backward requires [batch, heads, seq, dim]");
    const size_t b = s[0], h = s[1], n = s[2], d = s[3], bh = b * h;
    const Precision pr = q.precision();
    Tensor sc = Tensor::empty({bh, n, n}, Precision::FP32), p = Tensor::empty({bh, n, n}, pr);
    Tensor dp = Tensor::empty({bh, n, n}, Precision::FP32), ds = Tensor::empty({bh, n, n}, pr);
    AttentionGrads g{Tensor::empty(s, Precision::FP32), Tensor::empty(s, Precision::FP32), Tensor::empty(s, Precision::FP32)};
    check(it_attention_backward(Context::global().handle(), (it_dtype)pr, (int64_t)bh, (int64_t)n, (int64_t)d,
                                1.f / std::sqrt((float)d), 1, nullptr, nullptr, nullptr, grad_output.data(), q.data(),
                                k.data(), v.data(), (float *)sc.data(), p.data(), (float *)dp.data(), ds.data(),
                                (float *)g.dq.data(), (float *)g.dk.data(), (float *)g.dv.data()),
          "attention_backward");
    return g;
}

// attention_backward_recompute fused for head_dim 64 on [B,H,S,D]; deterministic (no atomics).
inline AttentionGrads flash_attention_backward(const Tensor &grad_output, const Tensor &q, const Tensor &k,
                                               const Tensor &v) {
    const auto &s = q.shape();
    detail::require(s.size() == 4, "attention_backward requires [batch, heads, seq, dim]");
    const size_t b = s[0], h = s[1], n = s[2], d = s[3];
    const Precision pr = q.precision();
    AttentionGrads g{Tensor::empty(s, Precision::FP32), Tensor::empty(s, Precision::FP32), Tensor::empty(s, Precision::FP32)};
    check(it_flash_attention_backward(Context::global().handle(), (it_dtype)pr, (int64_t)(b * h), (int64_t)n,
                                      (int64_t)d, 1.f / std::sqrt((float)d), 1, nullptr, nullptr, nullptr,
                                      grad_output.data(), q.data(), k.data(), v.data(), nullptr, nullptr,
                                      (float *)g.dq.data(), (float *)g.dk.data(), (float *)g.dv.data()),
          "attention_backward");
    return g;
}

// transpose_3d_gpu (src/ops/attention.rs:395-449; re-exported at src/ops/mod.rs:21):
// [batch, m, n] -> [batch, n, m], FP32, into a new tensor; panics on a size mismatch.
inline Tensor transpose_3d_gpu(const Tensor &t, size_t batch, size_t m, size_t n) {
    detail::require(t.numel() == batch * m * n, "assertion `left == right` failed: Tensor size mismatch");
    detail::require(t.is_f32(), "transpose_3d_gpu requires an FP32 tensor");
    Tensor out = Tensor::empty({batch, n, m}, Precision::FP32);
    check(it_transpose_3d(Context::global().handle(), (const float *)t.data(), (float *)out.data(), (int64_t)batch,
                          (int64_t)m, (int64_t)n),
          "transpose_3d_gpu");
    return out;
}

// causal_mask_3d_gpu (src/ops/attention.rs:455-517; re-exported at src/ops/mod.rs:21):
// [batch, seq, seq] with columns > row set to -inf, into a new FP32 tensor.
inline Tensor causal_mask_3d_gpu(const Tensor &t, size_t batch, size_t seq_len) {
    detail::require(t.numel() == batch * seq_len * seq_len, "assertion `left == right` failed: Tensor size mismatch");
    detail::require(t.is_f32(), "causal_mask_3d_gpu requires an FP32 tensor");
    Tensor out = Tensor::empty({batch, seq_len, seq_len}, Precision::FP32);
    check(it_causal_mask_3d(Context::global().handle(), (const float *)t.data(), (float *)out.data(),
                            (int64_t)batch, (int64_t)seq_len),
          "causal_mask_3d_gpu");
    return out;
}

// ------------------------------------------------------------------ training-step ops

namespace detail {
inline size_t last_dim(const Tensor &t) { return t.shape().empty() ? 1 : t.shape().back(); }
// Host index check as the reference asserts it (src/ops/embedding.rs:41-49), then upload as uint32.
inline Tensor upload_ids(const std::vector<uint32_t> &ids, size_t bound) {
    for (size_t i = 0; i < ids.size(); ++i)
        if (ids[i] >= bound)
            throw Panic("Index " + std::to_string(ids[i]) + " at position " + std::to_string(i) +
                        " is out of bounds for vocab_size " + std::to_string(bound));
    Tensor t = Tensor::empty({ids.size()}, Precision::FP32);  // raw 32-bit words
    if (!ids.empty()) check(it_memcpy_h2d(Context::global().handle(), t.data(), ids.data(), ids.size() * 4), "upload ids");
    return t;
}
}  // namespace detail

// rmsnorm (src/ops/norm.rs:31): y = x / sqrt(mean(x^2) + eps) * gamma over the last dimension.
inline Tensor rmsnorm(const Tensor &input, const Tensor &gamma, float eps) {
    if (!input.is_f32()) throw PrecisionMismatch("rmsnorm", "FP32", precision_name(input.precision()));
    const size_t dim = detail::last_dim(input);
    detail::require(gamma.numel() == dim, "gamma length must equal the last dimension");
    Tensor y = Tensor::empty(input.shape(), Precision::FP32);
    check(it_rmsnorm_forward(Context::global().handle(), IT_F32, (int64_t)(input.numel() / (dim ? dim : 1)),
                             (int64_t)dim, eps, (const float *)input.data(), nullptr, (const float *)gamma.data(),
                             nullptr, y.data()),
          "rmsnorm");
    return y;
}

// rmsnorm_backward (src/ops/backward/norm.rs:20) -> (grad_input, grad_gamma).
inline std::pair<Tensor, Tensor> rmsnorm_backward(const Tensor &grad_output, const Tensor &input, const Tensor &gamma,
                                                  float eps) {
    detail::require(grad_output.shape() == input.shape(), "grad_output and input shapes differ");
    const size_t dim = detail::last_dim(input);
    Tensor dx = Tensor::empty(input.shape(), Precision::FP32), dg = Tensor::empty({dim}, Precision::FP32);
    check(it_rmsnorm_backward(Context::global().handle(), (int64_t)(input.numel() / (dim ? dim : 1)), (int64_t)dim, eps,
                              (const float *)grad_output.data(), (const float *)input.data(),
                              (const float *)gamma.data(), nullptr, (float *)dx.data(), (float *)dg.data()),
          "rmsnorm_backward");
    return {dx, dg};
}

namespace detail {
inline Tensor rope(const Tensor &x, float base, size_t offset, int backward) {
    const auto &s = x.shape();
    require(s.size() == 4, "rope expects [batch, seq, heads, head_dim]");
    Tensor out = Tensor::empty(s, x.precision());
    const int64_t w = (int64_t)(s[2] * s[3]);
    check(it_rope(Context::global().handle(), (it_dtype)x.precision(), (it_dtype)x.precision(), (int64_t)s[0],
                  (int64_t)s[1], (int64_t)s[2], (int64_t)s[3], base, (int64_t)offset, backward, x.data(), w,
                  out.data(), w, 0),
          backward ? "rope_backward" : "rope");
    return out;
}
}  // namespace detail

// rope (src/ops/rope.rs:22) and rope_backward (src/ops/backward/rope.rs:16).
inline Tensor rope(const Tensor &input, float base, size_t position_offset) {
    return detail::rope(input, base, position_offset, 0);
}
inline Tensor rope_backward(const Tensor &grad_output, float base, size_t position_offset) {
    return detail::rope(grad_output, base, position_offset, 1);
}

// embedding (src/ops/embedding.rs:21): rows of weights [vocab, dim] by index, FP32 out.
inline Tensor embedding(const Tensor &weights, const std::vector<uint32_t> &indices) {
    detail::require(weights.shape().size() == 2, "Weights must be 2D [vocab_size, embed_dim]");
    const size_t vocab = weights.shape()[0], dim = weights.shape()[1];
    Tensor ids = detail::upload_ids(indices, vocab);
    Tensor out = Tensor::empty({indices.size(), dim}, Precision::FP32);
    check(it_embedding_forward(Context::global().handle(), (it_dtype)weights.precision(), IT_F32,
                               (int64_t)indices.size(), (int64_t)dim, (int64_t)vocab, weights.data(),
                               (const uint32_t *)ids.data(), out.data()),
          "embedding");
    return out;
}

// embedding_backward (src/ops/backward/embedding.rs:21): deterministic scatter-add.
inline Tensor embedding_backward(const Tensor &grad_output, const std::vector<uint32_t> &indices, size_t vocab_size) {
    detail::require(grad_output.is_f32(), "assertion `left == right` failed: embedding_backward requires FP32");
    detail::require(grad_output.shape().size() == 2, "grad_output must be 2D");
    const size_t n = grad_output.shape()[0], dim = grad_output.shape()[1];
    detail::require(indices.size() == n, "assertion `left == right` failed: indices length");
    Tensor ids = detail::upload_ids(indices, vocab_size);
    Tensor dw = Tensor::empty({vocab_size, dim}, Precision::FP32);
    check(it_embedding_backward(Context::global().handle(), (int64_t)n, (int64_t)dim, (int64_t)vocab_size,
                                (const float *)grad_output.data(), (const uint32_t *)ids.data(), (float *)dw.data()),
          "embedding_backward");
    return dw;
}

// cross_entropy_fused (src/ops/backward/loss.rs:248) -> (mean loss, losses [rows], grad [rows, vocab]).
struct CrossEntropy {
    float loss;
    Tensor losses, grad;
};
inline CrossEntropy cross_entropy_fused(const Tensor &logits, const std::vector<uint32_t> &targets) {
    detail::require(logits.is_f32(), "assertion `left == right` failed: cross_entropy_fused requires FP32");
    detail::require(logits.shape().size() == 2, "logits must be 2D");
    const size_t rows = logits.shape()[0], vocab = logits.shape()[1];
    detail::require(targets.size() == rows, "assertion `left == right` failed: targets length");
    CrossEntropy r{0.f, Tensor::zeros({rows}, Precision::FP32), Tensor::zeros({rows, vocab}, Precision::FP32)};
    if (rows == 0) return r;
    Tensor t = detail::upload_ids(targets, vocab);
    Tensor mean = Tensor::empty({1}, Precision::FP32);
    check(it_cross_entropy_fused(Context::global().handle(), IT_F32, (int64_t)rows, (int64_t)vocab,
                                 (const float *)logits.data(), (const uint32_t *)t.data(), (float *)r.losses.data(),
                                 r.grad.data(), (float *)mean.data()),
          "cross_entropy_fused");
    r.loss = mean.as_f32_slice()[0];
    return r;
}

// The loss half of cross_entropy_fused -> (mean loss, losses [rows], stats [rows, 2] = {max,
// 1 / sum exp(x - max)}); a GEMM with IT_EPI_XENT_A rebuilds the gradient from the stats.
struct CrossEntropyStats {
    float loss;
    Tensor losses, stats;
};
inline CrossEntropyStats cross_entropy_stats(const Tensor &logits, const std::vector<uint32_t> &targets) {
    detail::require(logits.is_f32(), "assertion `left == right` failed: cross_entropy_stats requires FP32");
    detail::require(logits.shape().size() == 2, "logits must be 2D");
    const size_t rows = logits.shape()[0], vocab = logits.shape()[1];
    detail::require(targets.size() == rows, "assertion `left == right` failed: targets length");
    CrossEntropyStats r{0.f, Tensor::zeros({rows}, Precision::FP32), Tensor::zeros({rows, 2}, Precision::FP32)};
    if (rows == 0) return r;
    Tensor t = detail::upload_ids(targets, vocab);
    Tensor mean = Tensor::empty({1}, Precision::FP32);
    check(it_cross_entropy_stats(Context::global().handle(), (int64_t)rows, (int64_t)vocab,
                                 (const float *)logits.data(), (const uint32_t *)t.data(), (float *)r.losses.data(),
                                 (float *)r.stats.data(), (float *)mean.data()),
          "cross_entropy_stats");
    r.loss = mean.as_f32_slice()[0];
    return r;
}

// swiglu_backward (src/ops/backward/elementwise.rs:149) -> (grad_gate, grad_up).
inline std::pair<Tensor, Tensor> swiglu_backward(const Tensor &grad_output, const Tensor &gate, const Tensor &up) {
    detail::require(grad_output.shape() == gate.shape() && gate.shape() == up.shape(), "swiglu_backward: shapes differ");
    const size_t cols = detail::last_dim(gate), rows = gate.numel() / (cols ? cols : 1);
    Tensor gg = Tensor::empty(gate.shape(), Precision::FP32), gu = Tensor::empty(gate.shape(), Precision::FP32);
    check(it_swiglu_backward(Context::global().handle(), (it_dtype)gate.precision(), IT_F32, (int64_t)rows,
                             (int64_t)cols, (const float *)grad_output.data(), (int64_t)cols, gate.data(), up.data(),
                             (int64_t)cols, gg.data(), gu.data(), (int64_t)cols),
          "swiglu_backward");
    return {gg, gu};
}

// total_l2_norm_gpu (src/ops/reduction.rs:94): sqrt of the summed squares of all tensors.
inline float total_l2_norm_gpu(const std::vector<const Tensor *> &tensors) {
    if (tensors.empty()) return 0.f;
    std::vector<const float *> p;
    std::vector<int64_t> n;
    for (const Tensor *t : tensors) {
        p.push_back((const float *)t->data());
        n.push_back((int64_t)t->numel());
    }
    Tensor out = Tensor::empty({2}, Precision::FP32);
    check(it_grad_norm_clip(Context::global().handle(), (int)p.size(), p.data(), n.data(),
                            std::numeric_limits<float>::infinity(), (float *)out.data()),
          "total_l2_norm_gpu");
    return out.as_f32_slice()[0];
}

// Lion (src/optim/lion/optimizer.rs:32-106; LionConfig defaults src/optim/lion/config.rs:91-99).
struct LionConfig {
    float lr = 1e-4f, beta1 = 0.9f, beta2 = 0.99f, weight_decay = 0.f;
};
struct ParamState {
    Tensor momentum;
    explicit ParamState(const Tensor &weights) : momentum(Tensor::zeros(weights.shape(), Precision::FP32)) {}
};
class Lion {
  public:
    explicit Lion(LionConfig c) : c_(c) {}
    static Lion with_lr(float lr) { return Lion(LionConfig{lr}); }
    float lr() const { return c_.lr; }
    void set_lr(float lr) { c_.lr = lr; }
    // Updates weights and state.momentum in place.
    void step(const Tensor &weights, const Tensor &gradients, ParamState &state) const {
        detail::require(weights.is_f32() && gradients.is_f32(), "lion: FP32 weights and gradients");
        detail::require(weights.numel() == gradients.numel(), "lion: weights and gradients differ in size");
        float *w = (float *)weights.data(), *m = (float *)state.momentum.data();
        const float *g = (const float *)gradients.data();
        const int64_t n = (int64_t)weights.numel();
        check(it_lion_step(Context::global().handle(), 1, &w, &m, &g, &n, c_.lr, c_.beta1, c_.beta2, c_.weight_decay,
                           nullptr, nullptr),
              "lion");
    }

  private:
    LionConfig c_;
};

// fused_rmsnorm_linear (src/ops/fused_rmsnorm_linear.rs:73-205): rmsnorm(input, gamma, eps) . weight^T
// without the normalized intermediate.
inline Tensor fused_rmsnorm_linear(const Tensor &input, const Tensor &gamma, const Tensor &weight, float eps) {
    detail::require(input.is_f32(), "assertion `left == right` failed: Input must be FP32");
    detail::require(input.shape().size() == 2, "Input must be 2D [batch_seq, hidden_dim]");
    detail::require(weight.shape().size() == 2, "Weight must be 2D [out_features, hidden_dim]");
    const size_t rows = input.shape()[0], hidden = input.shape()[1], out_f = weight.shape()[0];
    detail::require(weight.shape()[1] == hidden, "Hidden dimensions must match");
    detail::require(gamma.shape() == std::vector<size_t>{hidden}, "Gamma must have shape [hidden_dim]");
    Tensor out = Tensor::empty({rows, out_f}, Precision::FP32);
    check(it_fused_rmsnorm_linear(Context::global().handle(), (int64_t)rows, (int64_t)hidden, (int64_t)out_f, eps,
                                  (const float *)input.data(), (const float *)gamma.data(),
                                  (const float *)weight.data(), (float *)out.data()),
          "fused_rmsnorm_linear");
    return out;
}

// fused_linear_cross_entropy (src/ops/fused_linear_cross_entropy.rs:79-242): (mean loss, grad_hidden,
// grad_weight) without the [rows, vocab] logits; targets < 0 or >= vocab (-100) are ignored;
// grad_weight unscaled as in the reference. forward_only (:246-374) leaves grad_weight empty.
struct FusedLinearCE {
    float loss;
    Tensor grad_hidden;
    std::shared_ptr<Tensor> grad_weight;
};
inline FusedLinearCE fused_linear_cross_entropy(const Tensor &hidden, const Tensor &weight,
                                                const std::vector<int32_t> &targets, bool forward_only = false,
                                                int64_t chunk_bytes = 0) {
    detail::require(hidden.is_f32() && weight.is_f32(), "assertion `left == right` failed: FP32 required");
    detail::require(hidden.shape().size() == 2, "hidden must be 2D [batch*seq, hidden_dim]");
    detail::require(weight.shape().size() == 2, "weight must be 2D [vocab_size, hidden_dim]");
    const size_t rows = hidden.shape()[0], hd = hidden.shape()[1], vocab = weight.shape()[0];
    detail::require(weight.shape()[1] == hd, "weight hidden_dim must match hidden");
    detail::require(targets.size() == rows, "targets length must match batch*seq");
    detail::require(hd <= 256, "hidden_dim must be <= 256 for this kernel");
    FusedLinearCE r{0.f, Tensor::zeros({rows, hd}, Precision::FP32), nullptr};
    if (!forward_only) r.grad_weight = std::make_shared<Tensor>(Tensor::zeros({vocab, hd}, Precision::FP32));
    Tensor t = Tensor::empty({targets.size()}, Precision::FP32);  // raw int32 words
    if (!targets.empty())
        check(it_memcpy_h2d(Context::global().handle(), t.data(), targets.data(), targets.size() * 4), "upload targets");
    Tensor mean = Tensor::zeros({1}, Precision::FP32);
    check(it_fused_linear_cross_entropy(Context::global().handle(), (int64_t)rows, (int64_t)hd, (int64_t)vocab,
                                        (const float *)hidden.data(), (const float *)weight.data(),
                                        (const int32_t *)t.data(), nullptr, (float *)mean.data(),
                                        (float *)r.grad_hidden.data(),
                                        r.grad_weight ? (float *)r.grad_weight->data() : nullptr, chunk_bytes),
          "fused_linear_cross_entropy");
    r.loss = mean.as_f32_slice()[0];
    return r;
}

}  // namespace irontensor
