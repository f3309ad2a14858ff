// oxforge_net.hpp -- C++ host API of the OxideForge compute core.
//
// The reference's host side is Rust (src/cuda/runtime.rs, src/cuda/container,
// src/net).  No Rust toolchain exists in this build image, so the same API is
// kept here in C++ with the reference's names, argument meaning and order,
// over the C ABI of oxforge.h:
//   Rust                                 C++
//   CudaRuntime::new() -> Result         CudaRuntime::create()  (throws Error)
//   &mut CudaRuntime / &CudaRuntime      CudaRuntime&
//   Option<&CudaStream>                  const CudaStream* (nullptr = None)
//   Option<&Matrix> / Option<Vector>     const Matrix* / std::optional<Vector>
//   Matrix (owned, moved)                Matrix (move-only)
//   .unwrap() / assert! panics           throws oxforge::Error
// Dropping a DeviceBuffer (hence a Matrix or Vector) returns its memory to
// the runtime's exact-size pool instead of freeing it, so steady-state
// execution allocates nothing (the reference frees; runtime.rs:98-110 is its
// explicit recycle).
//
// MI355X-specific changes inside the executors (same results, fewer passes):
//   - Linear::forward is one GEMM with bias, residual and activation fused
//     into its epilogue (linear.rs:185-230 launches up to four kernels);
//   - transposed operands are read in place by NT/TN GEMMs instead of being
//     materialised (linear.rs:381-443, attention.rs:297-308, 366-398);
//   - Linear::learn fuses the lr scale and the subtraction into the dW GEMM;
//   - TrainingMlp keeps each layer's pre-activation from the forward pass
//     instead of recomputing it with an extra GEMM (mlp.rs:136-139).
// Extensions required by the benchmark configs: LayerNorm/RMSNorm gamma and
// beta (Normalization, attention.rs:147-175, has none), any row width
// (the reference asserts cols <= 1024) and explicit gradients
// (TrainingTransformer::backward_grads; the reference only applies SGD).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "oxforge.h"

namespace oxforge {

// ------------------------------------------------------------------ errors
class Error : public std::runtime_error {
public:
    Error(forge_status status, const std::string& what)
        : std::runtime_error(what), status_(status) {}
    forge_status status() const { return status_; }

private:
    forge_status status_;
};

void check(forge_status status, const char* what);

// BinaryOp (cuda.rs:3-10).
enum class BinaryOp : uint8_t { Add = 0, Sub = 1, Mul = 2, Div = 3 };

// InitType (runtime.rs:6-22): the four kinds as enumerators
// (InitType::Zero, ...) with the reference's is_zero().
class InitType {
public:
    enum Kind { Sequence, Reserve, Random, Zero };
    constexpr InitType(Kind kind) : kind_(kind) {}
    // runtime.rs:14-21: true for Zero only.
    constexpr bool is_zero() const { return kind_ == Zero; }
    constexpr operator Kind() const { return kind_; }

private:
    Kind kind_;
};

// NormType (transformer.rs:7-13); Layer is the default.
enum class NormType { Rms, Layer };

// Activation (linear.rs:12-19).
enum class Activation { Identity = 0, Gelu = 1, Relu = 2, Silu = 3 };

// Loss (mlp.rs:8-12).
enum class Loss { MeanSquaredError };

// ---------------------------------------------------------------- metadata
// The parameter descriptions of get_meta_data and the host copies of
// get_data (src/net/metadata.rs, linear.rs:79-114, mlp.rs:21-34, 99-119,
// transformer/inference.rs:12-24, 52-73): what the checkpoint writer
// serialises.  Byte ranges count f32 parameters in model order.

// metadata.rs:5-18.
struct MatrixMetadata {
    size_t rows = 0, cols = 0;
    uint64_t byte_start = 0, byte_end = 0;
    bool operator==(const MatrixMetadata& o) const {
        return rows == o.rows && cols == o.cols && byte_start == o.byte_start &&
               byte_end == o.byte_end;
    }
};
struct VectorMetadata {
    size_t len = 0;
    uint64_t byte_start = 0, byte_end = 0;
    bool operator==(const VectorMetadata& o) const {
        return len == o.len && byte_start == o.byte_start && byte_end == o.byte_end;
    }
};

// MetadataCursor (metadata.rs:20-68): hands out consecutive byte ranges of
// rows * cols (or len) f32 values from position 0.  An element or byte count
// that overflows throws Error (the reference panics).
class MetadataCursor {
public:
    MetadataCursor() = default;
    MatrixMetadata matrix(size_t rows, size_t cols);
    VectorMetadata vector(size_t len);
    uint64_t data_bytes() const { return position_; }

private:
    void reserve(size_t elements, uint64_t* start, uint64_t* end);
    uint64_t position_ = 0;
};

// HostData (metadata.rs:69-82): one parameter's values copied to the host.
class HostData {
public:
    explicit HostData(std::vector<float> values) : values_(std::move(values)) {}
    const std::vector<float>& values() const { return values_; }

private:
    std::vector<float> values_;
};

// linear.rs:79-86.
struct LinearMetadata {
    size_t input_neurons = 0, output_neurons = 0;
    Activation activation = Activation::Identity;
    MatrixMetadata weights;
    std::optional<VectorMetadata> bias;
};
// mlp.rs:21-34.
struct ResidualMetadata {
    size_t start = 0, end = 0;
};
struct MlpMetadata {
    size_t layer_count = 0;
    Loss loss = Loss::MeanSquaredError;
    std::optional<ResidualMetadata> residual;
    std::vector<LinearMetadata> layers;
};
// inference.rs:12-24, plus the gamma/beta extension: the norms' parameters,
// when a norm has them, after the output projection.
struct TransformerMetadata {
    size_t block_count = 1;
    bool attention_residual = true, feed_forward_residual = true;
    NormType normalization = NormType::Layer;
    MatrixMetadata position;
    LinearMetadata query, key, value;
    MlpMetadata feed_forward;
    LinearMetadata output;
    std::optional<VectorMetadata> norm1_gamma, norm1_beta, norm2_gamma, norm2_beta;
};

class CudaRuntime;

// A stream created by CudaRuntime::create_extra_streams.  Non-owning handle:
// the runtime destroys its streams.
class CudaStream {
public:
    explicit CudaStream(forge_stream* s = nullptr) : s_(s) {}
    forge_stream* raw() const { return s_; }

private:
    forge_stream* s_;
};

// DeviceBuffer<f32>: owns `len` floats from the runtime pool.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    DeviceBuffer(CudaRuntime* rt, forge_slice s) : rt_(rt), s_(s) {}
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : rt_(o.rt_), s_(o.s_) { o.s_ = forge_slice{nullptr, 0}; }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
    ~DeviceBuffer();

    size_t len() const { return s_.len; }
    bool is_empty() const { return s_.len == 0; }
    float* ptr() const { return s_.ptr; }
    forge_slice slice() const { return s_; }
    // Gives up ownership without returning the memory to the pool.
    forge_slice release() {
        forge_slice s = s_;
        s_ = forge_slice{nullptr, 0};
        return s;
    }

private:
    CudaRuntime* rt_ = nullptr;
    forge_slice s_{nullptr, 0};
};

// DeviceBuffer<u32> as CudaRuntime::get_u32_uninit_buffer returns it
// (runtime.rs:57-60): its own allocation, not pooled, released on drop.
class DeviceBufferU32 {
public:
    DeviceBufferU32() = default;
    DeviceBufferU32(CudaRuntime* rt, forge_slice_u32 s) : rt_(rt), s_(s) {}
    DeviceBufferU32(const DeviceBufferU32&) = delete;
    DeviceBufferU32& operator=(const DeviceBufferU32&) = delete;
    DeviceBufferU32(DeviceBufferU32&& o) noexcept : rt_(o.rt_), s_(o.s_) {
        o.s_ = forge_slice_u32{nullptr, 0};
    }
    DeviceBufferU32& operator=(DeviceBufferU32&& o) noexcept;
    ~DeviceBufferU32();

    size_t len() const { return s_.len; }
    bool is_empty() const { return s_.len == 0; }
    uint32_t* ptr() const { return s_.ptr; }
    forge_slice_u32 slice() const { return s_; }
    // to_host_vec (vector.rs:134); blocks until the copy is done.
    std::vector<uint32_t> to_host(CudaRuntime& rt) const;

private:
    CudaRuntime* rt_ = nullptr;
    forge_slice_u32 s_{nullptr, 0};
};

// ------------------------------------------------------------------ spans
// The closures the reference passes to for_each / map_sum (span.rs:261-299,
// elementwise.rs:70-79, reduction.rs:43-91) are device code compiled into
// its kernels; here they are the functor set of forge_map: x * p0, x + p0,
// GELU and its derivative, ReLU, SiLU (and derivatives), exp(x - p0),
// 0.5 x^2, identity.
struct MapFn {
    forge_map_op op;
    float p0;
    static MapFn scale(float v) { return {FORGE_MAP_SCALE, v}; }
    static MapFn add(float v) { return {FORGE_MAP_ADD, v}; }
    static MapFn exp_shift(float m) { return {FORGE_MAP_EXP_SHIFT, m}; }
    static MapFn half_square() { return {FORGE_MAP_HALF_SQ, 0.0f}; }
    static MapFn identity() { return {FORGE_MAP_IDENTITY, 0.0f}; }
    static MapFn of(forge_map_op op, float p0 = 0.0f) { return {op, p0}; }
};

class DeviceSpanMut;

// DeviceSpan<'a, f32> (span.rs:82-160): a non-owning, read-only view of
// `len` floats of a DeviceBuffer from `offset`.  Dropping it frees nothing;
// it must not outlive the buffer it views (the reference's borrow).
class DeviceSpan {
public:
    // span.rs:88-98 with check_range (span.rs:412-416): offset and
    // offset + len within the buffer, else Error (the reference panics).
    static DeviceSpan from_buffer(const DeviceBuffer& buffer, size_t offset, size_t len);
    // span.rs:120-122: the whole buffer in chunks of chunk_size (the last
    // may be shorter); chunk_size 0 is an Error.
    static std::vector<DeviceSpan> chunks(const DeviceBuffer& buffer, size_t chunk_size);

    size_t len() const { return s_.len; }
    bool is_empty() const { return s_.len == 0; }
    // The {ptr, len} kernel argument (DeviceSliceDescriptor, span.rs:7-11).
    forge_slice descriptor() const { return s_; }
    // Copies into a new pool buffer on the primary stream (span.rs:124-133).
    DeviceBuffer to_buffer(CudaRuntime& rt) const;
    DeviceBuffer to_buffer_async(CudaRuntime& rt) const;
    // Host scalars (span.rs:135-149, 301-359): empty spans give 0 (sum,
    // map_sum) and f32::MIN (max).
    float sum(CudaRuntime& rt) const;
    float max(CudaRuntime& rt) const;
    float map_sum(CudaRuntime& rt, MapFn f) const;

private:
    explicit DeviceSpan(forge_slice s) : s_(s) {}
    friend class DeviceSpanMut;
    forge_slice s_;
};

// DeviceSpanMut<'a, f32> (span.rs:161-299): the exclusive, writable view.
class DeviceSpanMut {
public:
    static DeviceSpanMut from_buffer(DeviceBuffer& buffer, size_t offset, size_t len);
    static std::vector<DeviceSpanMut> chunks(DeviceBuffer& buffer, size_t chunk_size);

    size_t len() const { return s_.len; }
    bool is_empty() const { return s_.len == 0; }
    forge_slice descriptor() const { return s_; }
    DeviceSpan into_span() const { return DeviceSpan(s_); }
    DeviceBuffer to_buffer(CudaRuntime& rt) const;
    DeviceBuffer to_buffer_async(CudaRuntime& rt) const;
    // x = f(x) in place (span.rs:245-279); nothing is launched when empty.
    void for_each(CudaRuntime& rt, MapFn f);
    void for_each_on(CudaRuntime& rt, const CudaStream* stream, MapFn f);
    void scale(float value, CudaRuntime& rt) { for_each(rt, MapFn::scale(value)); }
    float sum(CudaRuntime& rt) const { return into_span().sum(rt); }
    float max(CudaRuntime& rt) const { return into_span().max(rt); }
    float map_sum(CudaRuntime& rt, MapFn f) const { return into_span().map_sum(rt, f); }

private:
    explicit DeviceSpanMut(forge_slice s) : s_(s) {}
    forge_slice s_;
};

// VectorView<'a> (container.rs:17-19, vector_view.rs:6-47): a row of a
// Matrix (Matrix::row_views) or any span, with the Vector operations.
class VectorView {
public:
    explicit VectorView(DeviceSpanMut span) : span_(span) {}
    size_t len() const { return span_.len(); }
    void add_scalar(float value, CudaRuntime& rt) { span_.for_each(rt, MapFn::add(value)); }
    void scale(float value, CudaRuntime& rt) { span_.scale(value, rt); }
    void for_each(CudaRuntime& rt, MapFn f) { span_.for_each(rt, f); }
    float sum(CudaRuntime& rt) const { return span_.sum(rt); }
    float map_sum(CudaRuntime& rt, MapFn f) const { return span_.map_sum(rt, f); }
    // vector_view.rs:41-46: max, exp(x - max), sum, scale by 1 / sum.
    void softmax(CudaRuntime& rt);
    DeviceSpanMut& span() { return span_; }

private:
    DeviceSpanMut span_;
};

// ------------------------------------------------------------- containers
// Vector (container.rs:13-15, vector.rs, vector_runtime.rs).
class Vector {
public:
    Vector() = default;
    explicit Vector(DeviceBuffer b) : buffer_(std::move(b)) {}
    Vector(Vector&&) = default;
    Vector& operator=(Vector&&) = default;

    size_t len() const { return buffer_.len(); }
    // vector.rs:11-17.
    DeviceSpan as_span() const { return DeviceSpan::from_buffer(buffer_, 0, buffer_.len()); }
    DeviceSpan span(size_t offset, size_t len) const {
        return DeviceSpan::from_buffer(buffer_, offset, len);
    }
    std::vector<float> to_host(CudaRuntime& rt) const;
    void add_scalar(float value, CudaRuntime& rt);
    void scale(float value, CudaRuntime& rt);
    void scale_on(float value, CudaRuntime& rt, const CudaStream* stream);
    float sum(CudaRuntime& rt) const;
    float max(CudaRuntime& rt) const;
    void exp_shifted(float offset, CudaRuntime& rt);
    void softmax(CudaRuntime& rt);
    void binary_assign(const Vector& rhs, BinaryOp op, CudaRuntime& rt);
    void binary_assign_on(const Vector& rhs, BinaryOp op, CudaRuntime& rt,
                          const CudaStream* stream);
    float dot(const Vector& rhs, CudaRuntime& rt) const;
    // Vector::equals (vector.rs:117-136), comparing every element (the
    // reference kernel reduction.rs:132-174 only reports block 0).
    bool equals(const Vector& rhs, CudaRuntime& rt) const;

    forge_slice slice() const { return buffer_.slice(); }
    DeviceBuffer& buffer() { return buffer_; }
    const DeviceBuffer& buffer() const { return buffer_; }

private:
    DeviceBuffer buffer_;
};

// Matrix (container.rs:21-25, matrix.rs, norm.rs, rows.rs, convert.rs).
class Matrix {
public:
    Matrix() = default;
    Matrix(DeviceBuffer b, size_t rows, size_t cols)
        : buffer_(std::move(b)), rows_(rows), cols_(cols) {}
    Matrix(Matrix&&) = default;
    Matrix& operator=(Matrix&&) = default;

    std::vector<float> to_host(CudaRuntime& rt) const;
    // convert.rs:8-13: one view per row, in row order.
    std::vector<VectorView> row_views();
    size_t rows() const { return rows_; }
    size_t cols() const { return cols_; }
    size_t len() const { return buffer_.len(); }
    void scale(float value, CudaRuntime& rt);
    void add_scalar(float value, CudaRuntime& rt);
    void map(forge_map_op op, float p0, CudaRuntime& rt, const CudaStream* stream = nullptr);
    void binary_assign(const Matrix& rhs, BinaryOp op, CudaRuntime& rt);
    void binary_assign_on(const Matrix& rhs, BinaryOp op, CudaRuntime& rt,
                          const CudaStream* stream);
    void causal_mask(CudaRuntime& rt);
    void softmax_rows(CudaRuntime& rt);
    // The gamma/beta overloads are the affine extension (nullptr = the
    // reference's parameterless kernels, norm.rs:26-69).
    void layer_norm(CudaRuntime& rt, const Vector* gamma = nullptr, const Vector* beta = nullptr);
    void rms_norm(CudaRuntime& rt, const Vector* gamma = nullptr);
    void binary_assign_by_rows(const Vector& vec, BinaryOp op, CudaRuntime& rt);
    void binary_assign_by_rows_on(const Vector& vec, BinaryOp op, CudaRuntime& rt,
                                  const CudaStream* stream);

    forge_slice slice() const { return buffer_.slice(); }
    DeviceBuffer& buffer() { return buffer_; }
    const DeviceBuffer& buffer() const { return buffer_; }
    DeviceBuffer into_buffer() { return std::move(buffer_); }

private:
    DeviceBuffer buffer_;
    size_t rows_ = 0, cols_ = 0;
};

// ----------------------------------------------------------------- runtime
// CudaRuntime (runtime.rs:24-212) with the container constructors of
// matrix.rs:95-326, norm.rs:72-159, rows.rs:45-89, convert.rs:16-151 and
// vector_runtime.rs:9-118.
class CudaRuntime {
public:
    static std::unique_ptr<CudaRuntime> create(int device = 0, const char* module_path = nullptr);
    // Wraps an existing C runtime without taking ownership.
    static std::unique_ptr<CudaRuntime> borrow(forge_runtime* rt);
    ~CudaRuntime();
    CudaRuntime(const CudaRuntime&) = delete;
    CudaRuntime& operator=(const CudaRuntime&) = delete;

    forge_runtime* raw() const { return rt_; }

    DeviceBuffer get_uninit_buffer(size_t size);
    // runtime.rs:57-60: an uninitialised u32 buffer (not from the pool).
    DeviceBufferU32 get_u32_uninit_buffer(size_t size);
    DeviceBuffer get_zerod_buffer(size_t size);
    void reserve_buffers(size_t size, size_t count);
    void recycle_buffer(DeviceBuffer&& buffer);
    void sync();
    // The primary stream is represented by nullptr in every *_on call.
    const CudaStream* stream() const { return nullptr; }
    std::vector<CudaStream> create_extra_streams(size_t count);
    void fork_streams(const std::vector<CudaStream>& streams);
    void join_streams(const std::vector<CudaStream>& streams);
    void sync_streams(const std::vector<CudaStream>& streams);
    // `waiter` waits on everything queued on the primary stream
    // (CudaStream::join(primary), e.g. linear.rs:126).
    void stream_join_primary(const CudaStream* waiter);
    DeviceBuffer concat_buffers(const std::vector<const DeviceBuffer*>& buffers);
    // span.rs:483-523: the spans' elements back to back in a new buffer.
    DeviceBuffer concat_buffers_from_span(const std::vector<DeviceSpan>& spans);
    DeviceBuffer clone_buffer(const DeviceBuffer& buffer);
    // runtime.rs:184-186: the span's elements in a new pool buffer, copied
    // on the primary stream (span.to_buffer_async).
    DeviceBuffer span_to_buffer_async(const DeviceSpan& span);

    // Matrix constructors and operations.
    Matrix matrix_from_host(const std::vector<float>& values, size_t rows, size_t cols);
    Matrix matrix_from_host(const float* values, size_t rows, size_t cols);
    Matrix matrix_from_device(forge_slice values, size_t rows, size_t cols);
    Matrix matrix_multiply(const Matrix& a, const Matrix& b);
    Matrix matrix_multiply_on(const CudaStream* stream, const Matrix& a, const Matrix& b);
    void matrix_multiply_into_on(const CudaStream* stream, const Matrix& a, const Matrix& b,
                                 Matrix& result);
    Matrix matrix_add(const Matrix& a, const Matrix& b);
    Matrix matrix_sub(const Matrix& a, const Matrix& b);
    Matrix matrix_mul(const Matrix& a, const Matrix& b);
    Matrix matrix_div(const Matrix& a, const Matrix& b);
    Matrix matrix_binary(const Matrix& a, const Matrix& b, BinaryOp op);
    Matrix matrix_binary_on(const CudaStream* stream, const Matrix& a, const Matrix& b,
                            BinaryOp op);
    void recycle_matrix(Matrix&& m);
    Matrix new_matrix(InitType init, size_t rows, size_t cols);
    Matrix new_uninit_matrix(size_t rows, size_t cols);
    Matrix clone_matrix(const Matrix& m);
    Matrix clone_matrix_on(const Matrix& m, const CudaStream* stream);
    Matrix softmax_rows_backward(const Matrix& probabilities, const Matrix& output_gradient);
    Matrix layer_norm_backward(const Matrix& input, const Matrix& output_gradient,
                               const Vector* gamma = nullptr, Vector* dgamma = nullptr,
                               Vector* dbeta = nullptr);
    Matrix rms_norm_backward(const Matrix& input, const Matrix& output_gradient,
                             const Vector* gamma = nullptr, Vector* dgamma = nullptr);
    Vector matrix_sum_rows(const Matrix& m);
    Vector matrix_sum_rows_on(const Matrix& m, const CudaStream* stream);
    // Column sums (the reference's transpose + sum_rows, linear.rs:267-272).
    Vector matrix_sum_cols(const Matrix& m, const CudaStream* stream = nullptr);
    Matrix matrix_transpose(const Matrix& m);
    Matrix matrix_transpose_on(const Matrix& m, const CudaStream* stream);
    Matrix vector_zip(const std::vector<Vector>& vecs);
    std::vector<Vector> matrix_split(const Matrix& m);
    Matrix broadcast(const Vector& v, size_t copies);
    Vector extract_vector(Matrix&& m);
    std::vector<Matrix> matrix_slice(const Matrix& m, size_t cols, size_t rows);
    Vector matrix_into_vector(Matrix&& m);
    Matrix vector_into_matrix(Vector&& v);

    // Vector constructors and operations.
    Vector vector_from_host(const std::vector<float>& values);
    Vector vector_from_host(const float* values, size_t n);
    Vector vector_from_device(forge_slice values);
    void recycle_vector(Vector&& v);
    Vector new_vector(InitType init, size_t size);
    Vector clone_vector(const Vector& v);
    Vector clone_vector_on(const Vector& v, const CudaStream* stream);
    Vector vector_add(const Vector& a, const Vector& b);
    Vector vector_sub(const Vector& a, const Vector& b);
    Vector vector_mul(const Vector& a, const Vector& b);
    Vector vector_div(const Vector& a, const Vector& b);
    Vector vector_binary(const Vector& a, const Vector& b, BinaryOp op);

    // Fused GEMM (forge_gemm_ex_f32) used by the executors.
    void gemm_ex(const CudaStream* stream, bool trans_a, bool trans_b, const Matrix& a,
                 const Matrix& b, forge_slice c, size_t m, size_t n, size_t k,
                 const forge_gemm_epilogue& ep);

private:
    explicit CudaRuntime(forge_runtime* rt, bool owned) : rt_(rt), owned_(owned) {}
    forge_runtime* rt_;
    bool owned_;
    std::vector<forge_stream*> streams_;
};

forge_stream* stream_raw(const CudaStream* s);
forge_gemm_epilogue plain_epilogue();

// -------------------------------------------------------------- executors

// Linear (linear.rs:72-532).  weights is [input_neurons, output_neurons].
class Linear {
public:
    Linear(Matrix weights, std::optional<Vector> bias, Activation activation);

    // linear.rs:97-105: shapes, activation and the byte ranges of the
    // weights, then the bias when there is one.
    LinearMetadata get_meta_data(MetadataCursor& cursor) const;
    // linear.rs:107-114: host copies of the weights and the bias (if any).
    std::vector<HostData> get_data(CudaRuntime& rt) const;

    Matrix forward(const Matrix& input, const Matrix* residual, CudaRuntime& rt,
                   const CudaStream* stream);
    Matrix affine(const Matrix& input, const Matrix* residual, CudaRuntime& rt,
                  const CudaStream* stream);
    void activate(Matrix& output, CudaRuntime& rt, const CudaStream* stream);
    // (gradient, bias_gradient): gradient = dY * act'(pre_activation).
    std::pair<Matrix, std::optional<Vector>> backward(const Matrix* pre_activation,
                                                      const Matrix& output_gradient,
                                                      CudaRuntime& rt, const CudaStream* stream);
    bool needs_pre_activation() const { return activation_ != Activation::Identity; }
    static Vector loss_rows(const Matrix& output, const Matrix& target, CudaRuntime& rt,
                            const CudaStream* stream);
    // W -= lr * input^T gradient; b -= lr * bias_gradient.
    void learn(const Matrix& input, const Matrix& gradient, const Vector* bias_gradient,
               float learning_rate, CudaRuntime& rt, const CudaStream* stream);
    // gradient * W^T.
    Matrix input_gradient(const Matrix& gradient, CudaRuntime& rt, const CudaStream* stream);
    std::pair<Matrix, std::optional<Vector>> backward_with_res(
        const Matrix& pre_activation, const Matrix& output_gradient,
        const Matrix& residual_gradient, CudaRuntime& rt, const CudaStream* stream);

    // Extensions used by the executors.
    // forward that also stores the pre-activation (nullptr to skip).
    Matrix forward_keep(const Matrix& input, const Matrix* residual, Matrix* pre_activation,
                        CudaRuntime& rt, const CudaStream* stream);
    // forward into a caller-owned output (Linear::forward_on, linear.rs:145-155).
    void forward_into(const Matrix& input, const Matrix* residual, Matrix& output,
                      CudaRuntime& rt, const CudaStream* stream,
                      Matrix* pre_activation = nullptr);
    // The GEMM of forward_into as a batch entry (bias and activation fused).
    forge_gemm_problem forward_problem(const Matrix& input, Matrix& output) const;
    // The weight-update GEMM of learn_keep as a batch entry (W -= lr X^T G,
    // dW into *weight_gradient when given); the bias is not touched.
    forge_gemm_problem learn_problem(const Matrix& input, const Matrix& gradient,
                                     float learning_rate, Matrix* weight_gradient);
    // learn that also stores dW (and db) when given, for explicit gradients.
    void learn_keep(const Matrix& input, const Matrix& gradient, const Vector* bias_gradient,
                    float learning_rate, Matrix* weight_gradient, CudaRuntime& rt,
                    const CudaStream* stream, bool bias_step = true);
    // learn_keep with the bias gradient formed here: the weight update as a
    // fused GEMM, then the column sums of `gradient` and the bias's SGD step
    // in one pass (forge_sum_cols_sgd); the sums are kept in
    // *bias_gradient_out when given.  Same results as computing the bias
    // gradient first and calling learn_keep.
    void learn_from_gradient(const Matrix& input, const Matrix& gradient, float learning_rate,
                             Matrix* weight_gradient, std::optional<Vector>* bias_gradient_out,
                             CudaRuntime& rt, const CudaStream* stream);
    // input_gradient accumulated onto `accumulate` (dX + accumulate, one
    // rounded add per element, written into `accumulate`).
    void input_gradient_accumulate(const Matrix& gradient, Matrix& accumulate, CudaRuntime& rt,
                                   const CudaStream* stream);

    const Matrix& weights() const { return weights_; }
    const std::optional<Vector>& bias() const { return bias_; }
    Activation activation() const { return activation_; }
    Matrix& weights_mut() { return weights_; }
    std::optional<Vector>& bias_mut() { return bias_; }

private:
    Matrix weights_;
    std::optional<Vector> bias_;
    Activation activation_;
};

// MlpExecutor (mlp.rs:14-169).  res_range = [start, end): residual from the
// input of layer `start` to the output of layer `end - 1`.
class MlpExecutor {
public:
    MlpExecutor(std::vector<Linear> layers, std::optional<std::pair<size_t, size_t>> res_range,
                Loss loss = Loss::MeanSquaredError);
    // mlp.rs:37-51 (MlpExecutor::new is the constructor with the default
    // loss): at least one layer, and start < end <= layers for a residual.
    static MlpExecutor with_loss(std::vector<Linear> layers,
                                 std::optional<std::pair<size_t, size_t>> res_range, Loss loss) {
        return MlpExecutor(std::move(layers), res_range, loss);
    }
    // mlp.rs:99-112: layer count, loss, residual range, then each layer's
    // metadata in order.
    MlpMetadata get_meta_data(MetadataCursor& cursor) const;
    // mlp.rs:114-119: every layer's get_data, in order.
    std::vector<HostData> get_data(CudaRuntime& rt) const;
    Matrix forward(const Matrix& input, CudaRuntime& rt);
    // forward with an extra residual added to the final layer's output
    // (fused into its epilogue); used by the transformer blocks.
    Matrix forward_plus(const Matrix& input, const Matrix* final_residual, CudaRuntime& rt);
    size_t len() const { return layers_.size(); }
    bool is_empty() const { return layers_.empty(); }
    Loss loss() const { return loss_; }
    // layer_inputs[i] is the input of layer i; pre_activations[i] the cached
    // pre-activation of layer i (empty Matrix when not needed / not cached).
    Matrix backward(const std::vector<Matrix>& layer_inputs,
                    const std::vector<Matrix>& pre_activations, const Matrix& output_gradient,
                    float learning_rate, CudaRuntime& rt,
                    std::vector<Matrix>* weight_gradients = nullptr,
                    std::vector<std::optional<Vector>>* bias_gradients = nullptr,
                    const Matrix* input_gradient_residual = nullptr);
    std::vector<Linear>& layers() { return layers_; }
    const std::vector<Linear>& layers() const { return layers_; }
    std::optional<std::pair<size_t, size_t>> res_range() const { return res_range_; }

private:
    std::vector<Linear> layers_;
    std::optional<std::pair<size_t, size_t>> res_range_;
    Loss loss_;
};

// InferenceMLP (mlp.rs:171-201).
class InferenceMLP {
public:
    InferenceMLP(std::vector<Linear> layers, std::optional<std::pair<size_t, size_t>> res_range,
                 Loss loss = Loss::MeanSquaredError)
        : executor_(std::move(layers), res_range, loss) {}
    // mlp.rs:180-184.
    static InferenceMLP with_loss(std::vector<Linear> layers,
                                  std::optional<std::pair<size_t, size_t>> res_range, Loss loss) {
        return InferenceMLP(std::move(layers), res_range, loss);
    }
    // mlp.rs:186-192.
    MlpMetadata get_meta_data(MetadataCursor& cursor) const {
        return executor_.get_meta_data(cursor);
    }
    std::vector<HostData> get_data(CudaRuntime& rt) const { return executor_.get_data(rt); }
    Loss loss() const { return executor_.loss(); }
    Matrix forward(const Matrix& input, CudaRuntime& rt) { return executor_.forward(input, rt); }
    MlpExecutor& executor() { return executor_; }
    const MlpExecutor& executor() const { return executor_; }

private:
    MlpExecutor executor_;
};

// TrainingMlp (mlp.rs:203-269): keeps each layer's input (and, here, its
// pre-activation) for backward.
class TrainingMlp {
public:
    TrainingMlp(std::vector<Linear> layers, std::optional<std::pair<size_t, size_t>> res_range,
                Loss loss = Loss::MeanSquaredError)
        : executor_(std::move(layers), res_range, loss) {}
    // mlp.rs:214-219.
    static TrainingMlp with_loss(std::vector<Linear> layers,
                                 std::optional<std::pair<size_t, size_t>> res_range, Loss loss) {
        return TrainingMlp(std::move(layers), res_range, loss);
    }
    // mlp.rs:221-228.
    MlpMetadata get_meta_data(MetadataCursor& cursor) const {
        return executor_.get_meta_data(cursor);
    }
    std::vector<HostData> get_data(CudaRuntime& rt) const { return executor_.get_data(rt); }
    Loss loss() const { return executor_.loss(); }
    Matrix forward(Matrix input, CudaRuntime& rt);
    // forward whose output also adds the MLP's own input (fused into the
    // last layer's epilogue) when add_input_to_output is set.
    Matrix forward_plus(Matrix input, bool add_input_to_output, CudaRuntime& rt);
    Matrix backward(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt);
    Matrix backward_grads(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt,
                          std::vector<Matrix>* weight_gradients,
                          std::vector<std::optional<Vector>>* bias_gradients,
                          const Matrix* input_gradient_residual);
    const Matrix* input() const { return layer_inputs_.empty() ? nullptr : &layer_inputs_[0]; }
    MlpExecutor& executor() { return executor_; }
    const MlpExecutor& executor() const { return executor_; }

private:
    std::vector<Matrix> layer_inputs_;
    std::vector<Matrix> pre_activations_;
    MlpExecutor executor_;
};

// Normalization (attention.rs:147-175) with the gamma/beta extension.
struct Normalization {
    NormType kind = NormType::Layer;
    std::optional<Vector> gamma;  // absent: the reference's parameterless norm
    std::optional<Vector> beta;   // LayerNorm only
    float eps = 1e-5f;            // norm.rs:45,66,123,153
    void forward(Matrix& m, CudaRuntime& rt) const;
    // The same normalisation written to dst (dst == src is the in-place call).
    void forward_into(const Matrix& src, Matrix& dst, CudaRuntime& rt) const;
    Matrix backward(const Matrix& input, const Matrix& output_gradient, CudaRuntime& rt,
                    Vector* dgamma = nullptr, Vector* dbeta = nullptr) const;
    // backward, then the SGD step of this norm's gamma/beta (when present)
    // in the same final pass; dgamma/dbeta optional gradient outputs.  With
    // dot_sub and dot, also dot[r] = dot_scale * sum_c dx[r,c] *
    // (input[r,c] - dot_sub[r,c]) (forge_layer_norm_bwd_sgd_dot).
    Matrix backward_step(const Matrix& input, const Matrix& output_gradient, float learning_rate,
                         CudaRuntime& rt, Vector* dgamma = nullptr, Vector* dbeta = nullptr,
                         const Matrix* dot_sub = nullptr, Vector* dot = nullptr,
                         float dot_scale = 1.0f);
};

// QkvProjection (attention.rs:15-144).  With `streams` (three streams of
// CudaRuntime::create_extra_streams) the three projections run as the
// reference runs them: the streams fork from the primary stream, Q, K and V
// each run on their own stream, wait_for_query_key joins the first two and
// wait_for_value the third.  Without streams they are one batched GEMM
// launch on the primary stream (three launches when the shapes differ):
// the faster choice on MI355X, where a cross-queue fork costs about 24 us
// and a join about 7 us of idle device.  Both give bit-identical results.
class QkvProjection {
public:
    QkvProjection(Linear query, Linear key, Linear value,
                  std::optional<std::vector<CudaStream>> streams);
    struct Projected {
        Matrix query, key, value;
    };
    Projected project(const Matrix& query_input, const Matrix& key_value_input, CudaRuntime& rt);
    void wait_for_query_key(CudaRuntime& rt);
    void wait_for_value(CudaRuntime& rt);
    Linear& query() { return query_; }
    Linear& key() { return key_; }
    Linear& value() { return value_; }
    const Linear& query() const { return query_; }
    const Linear& key() const { return key_; }
    const Linear& value() const { return value_; }

private:
    Linear query_, key_, value_;
    std::optional<std::vector<CudaStream>> streams_;
    bool joined_qk_ = true, joined_v_ = true;  // no projection pending on the streams
};

// Gradients of the single-head Post-Norm block (the explicit-gradient
// extension).  Linear order: query, key, value, ffn layers..., output.
struct TransformerGrads {
    std::vector<Matrix> weights;
    std::vector<std::optional<Vector>> biases;
    std::optional<Vector> norm1_gamma, norm1_beta, norm2_gamma, norm2_beta;
    Matrix position;  // also the input gradient (input and position enter as X + P)
};

// Attention (attention.rs:177-401).
class Attention {
public:
    Attention(Linear query, Linear key, Linear value,
              std::optional<std::vector<CudaStream>> streams, Normalization norm);
    NormType norm_type() const { return norm_.kind; }
    Matrix forward(const Matrix& query_input, const Matrix& key_value_input, CudaRuntime& rt);
    Matrix forward_mask(const Matrix& query_input, const Matrix& key_value_input,
                        CudaRuntime& rt);
    Matrix forward_self_training(Matrix input, CudaRuntime& rt);
    // The attention output before its norm (X + A, attention.rs:243-253),
    // with row_sumsq [rows, ceil(cols / 32)] receiving each row's sums of
    // squares over 32-column blocks (forge_gemm_epilogue row_sumsq_out), so
    // that a parameterless RMSNorm can be folded into the next product.
    Matrix forward_pre_norm(const Matrix& query_input, const Matrix& key_value_input, bool mask,
                            Matrix& row_sumsq, CudaRuntime& rt);
    // With `input_gradient` given, the returned gradient is written there
    // (same shape as the attention input) and an empty Matrix is returned.
    // With `position` given (the training block's position matrix, same
    // shape), the product that completes the input gradient dXp also applies
    // position -= learning_rate * dXp (encoder.rs:180-184) in its epilogue.
    Matrix backward_self(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt,
                         TransformerGrads* grads = nullptr, Matrix* input_gradient = nullptr,
                         Matrix* position = nullptr);
    void normalize(Matrix& m, CudaRuntime& rt, const Normalization* norm = nullptr) const;
    Normalization& normalization() { return norm_; }
    QkvProjection& qkv() { return qkv_; }
    const Normalization& normalization() const { return norm_; }
    const QkvProjection& qkv() const { return qkv_; }
    // Largest score matrix (bytes) held at once.  A [S, Sk] score matrix
    // above it is never formed: the scores, probabilities and their
    // gradients are computed for one chunk of query rows at a time (a
    // multiple of 64 rows, at least 64), and the training step recomputes
    // each chunk's probabilities in backward instead of caching S x Sk.
    // Default 1 GiB (S = Sk = 16384 still unchunked).
    void set_max_score_bytes(size_t bytes) { max_score_bytes_ = bytes; }
    size_t max_score_bytes() const { return max_score_bytes_; }

private:
    Matrix attention_value(QkvProjection::Projected projected, const Matrix& residual, bool mask,
                           CudaRuntime& rt, Matrix* row_sumsq = nullptr);
    // out = softmax(scale Q K^T (masked)) V + residual in query chunks.
    void chunked_forward(const Matrix& q, const Matrix& k, const Matrix& v,
                         const Matrix& residual, bool mask, size_t chunk, Matrix& out,
                         CudaRuntime& rt, Matrix* row_sumsq = nullptr);
    struct Cache {
        Matrix input, query, key, value, probabilities, pre_norm;
    };
    QkvProjection qkv_;
    Normalization norm_;
    std::optional<Cache> cache_;
    size_t max_score_bytes_ = size_t(1) << 30;
};

// InferenceBlock (inference.rs:26-108).
class InferenceBlock {
public:
    InferenceBlock(Linear query, Linear key, Linear value, Matrix position, InferenceMLP fcs,
                   Linear output, std::optional<std::vector<CudaStream>> qkv_streams,
                   NormType norm_type, std::optional<Normalization> norm2 = std::nullopt);
    Matrix forward(const Matrix& input, CudaRuntime& rt);
    Matrix forward_mask(const Matrix& input, CudaRuntime& rt);
    // The same, with the output projection written into `output`.
    void forward_into(const Matrix& input, Matrix& output, CudaRuntime& rt, bool mask = false);
    // inference.rs:52-73: Q, K, V, position, the feed-forward layers and the
    // output projection, in that order (then the norms' gamma/beta, the
    // extension, when present).
    TransformerMetadata get_meta_data(MetadataCursor& cursor) const;
    std::vector<HostData> get_data(CudaRuntime& rt) const;
    // With both norms the reference's parameterless RMSNorm and a feed-forward
    // network without an inner residual range, the forward folds each norm
    // into the products on either side of it (on by default): the
    // attention-value product and the last feed-forward layer also write the
    // rows' sums of squares; the first feed-forward layer and the output
    // projection divide their products by the rows' RMS, and the last layer
    // divides its residual.  Two kernels and their launch boundaries go; the
    // results agree with the reference's order (normalise, then multiply) to
    // within rounding.  Off: the reference's launch order.
    void set_fold_norms(bool on) { fold_norms_ = on; }
    bool fold_norms() const { return fold_norms_; }
    bool can_fold_norms() const;
    Attention& attention() { return attention_; }
    Normalization& norm2() { return norm2_; }
    Matrix& position() { return position_; }
    InferenceMLP& fcs() { return fcs_; }
    Linear& output() { return output_; }

private:
    Matrix finish_forward(Matrix positioned, Matrix x, CudaRuntime& rt, Matrix* target);
    Matrix forward_folded(const Matrix& input, bool mask, CudaRuntime& rt, Matrix* target);
    Attention attention_;
    Matrix position_;
    InferenceMLP fcs_;
    Linear output_;
    Normalization norm2_;
    bool fold_norms_ = true;
};

namespace encoder {
// encoder::InferenceTransformer (encoder.rs:16-56).
class InferenceTransformer {
public:
    InferenceTransformer(Linear q, Linear k, Linear v, Matrix position, InferenceMLP fcs,
                         Linear output, std::optional<std::vector<CudaStream>> qkv_streams,
                         NormType norm_type, std::optional<Normalization> norm1 = std::nullopt,
                         std::optional<Normalization> norm2 = std::nullopt);
    Matrix forward(const Matrix& input, CudaRuntime& rt) { return block_.forward(input, rt); }
    void forward_into(const Matrix& input, Matrix& output, CudaRuntime& rt) {
        block_.forward_into(input, output, rt, false);
    }
    // encoder.rs:45-51.
    TransformerMetadata get_meta_data(MetadataCursor& cursor) const {
        return block_.get_meta_data(cursor);
    }
    std::vector<HostData> get_data(CudaRuntime& rt) const { return block_.get_data(rt); }
    InferenceBlock& block() { return block_; }

private:
    InferenceBlock block_;
};

// encoder::TrainingTransformer (encoder.rs:58-186).
class TrainingTransformer {
public:
    TrainingTransformer(Linear q, Linear k, Linear v, Matrix position, TrainingMlp fcs,
                        Linear output, NormType norm_type,
                        std::optional<Normalization> norm1 = std::nullopt,
                        std::optional<Normalization> norm2 = std::nullopt);
    Matrix forward(const Matrix& input, CudaRuntime& rt);
    // The same, with the output projection written into `output`.
    void forward_into(const Matrix& input, Matrix& output, CudaRuntime& rt);
    // Gradients, then SGD with learning_rate (reference semantics).
    Matrix backward(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt);
    // Same update, and every gradient exposed in `grads`.
    Matrix backward_grads(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt,
                          TransformerGrads& grads);
    // backward / backward_grads (grads may be null) with the input gradient
    // written into `input_gradient` ([seq, hidden]) instead of a new matrix.
    void backward_into(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt,
                       Matrix& input_gradient, TransformerGrads* grads = nullptr);
    // encoder.rs:90-112 (the same layout as the inference block).
    TransformerMetadata get_meta_data(MetadataCursor& cursor) const;
    std::vector<HostData> get_data(CudaRuntime& rt) const;
    Attention& attention() { return attention_; }
    TrainingMlp& fcs() { return fcs_; }
    Linear& output() { return output_; }
    Matrix& position() { return position_; }
    Normalization& norm2() { return norm2_; }

private:
    Matrix backward_impl(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt,
                         TransformerGrads* grads, Matrix* input_gradient = nullptr);
    struct Cache {
        Matrix second_pre_norm, encoded;
    };
    Attention attention_;
    Matrix position_;
    TrainingMlp fcs_;
    Linear output_;
    Normalization norm2_;
    std::optional<Cache> cache_;
};
}  // namespace encoder

namespace decoder {
// decoder::InferenceTransformer (decoder.rs:13-53): the causal-mask block.
class InferenceTransformer {
public:
    InferenceTransformer(Linear q, Linear k, Linear v, Matrix position, InferenceMLP fcs,
                         Linear output, std::optional<std::vector<CudaStream>> qkv_streams,
                         NormType norm_type)
        : block_(std::move(q), std::move(k), std::move(v), std::move(position), std::move(fcs),
                 std::move(output), std::move(qkv_streams), norm_type) {}
    Matrix forward(const Matrix& input, CudaRuntime& rt) { return block_.forward_mask(input, rt); }
    void forward_into(const Matrix& input, Matrix& output, CudaRuntime& rt) {
        block_.forward_into(input, output, rt, true);
    }
    // decoder.rs:42-48.
    TransformerMetadata get_meta_data(MetadataCursor& cursor) const {
        return block_.get_meta_data(cursor);
    }
    std::vector<HostData> get_data(CudaRuntime& rt) const { return block_.get_data(rt); }
    InferenceBlock& block() { return block_; }

private:
    InferenceBlock block_;
};
}  // namespace decoder

}  // namespace oxforge
