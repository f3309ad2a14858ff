// host_api.cpp -- CudaRuntime, Matrix, Vector and DeviceBuffer over the C ABI.
//
// Mirrors src/cuda/runtime.rs, src/cuda/span.rs and src/cuda/container/*.rs.
// Every device operation is one call into include/oxforge.h; shape checks
// that the reference makes with assert! throw oxforge::Error here.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <random>

#include "oxforge_net.hpp"

namespace oxforge {

void check(forge_status status, const char* what) {
    if (status != FORGE_OK)
        throw Error(status, std::string(what) + ": " + forge_last_error());
}

static void require(bool cond, const char* what) {
    if (!cond) throw Error(FORGE_EINVAL, std::string("assertion failed: ") + what);
}

forge_stream* stream_raw(const CudaStream* s) { return s ? s->raw() : nullptr; }

forge_gemm_epilogue plain_epilogue() {
    forge_gemm_epilogue ep;
    std::memset(&ep, 0, sizeof ep);
    ep.alpha = 1.0f;
    ep.activation = FORGE_ACT_IDENTITY;
    ep.aux_activation = FORGE_ACT_IDENTITY;
    return ep;
}

// ---------------------------------------------------------------- buffers

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
        if (rt_ && s_.ptr) (void)forge_recycle(rt_->raw(), s_);
        rt_ = o.rt_;
        s_ = o.s_;
        o.s_ = forge_slice{nullptr, 0};
    }
    return *this;
}

DeviceBuffer::~DeviceBuffer() {
    if (rt_ && s_.ptr) (void)forge_recycle(rt_->raw(), s_);
}

DeviceBufferU32& DeviceBufferU32::operator=(DeviceBufferU32&& o) noexcept {
    if (this != &o) {
        if (rt_ && s_.ptr) (void)forge_free_u32(rt_->raw(), s_);
        rt_ = o.rt_;
        s_ = o.s_;
        o.s_ = forge_slice_u32{nullptr, 0};
    }
    return *this;
}

DeviceBufferU32::~DeviceBufferU32() {
    if (rt_ && s_.ptr) (void)forge_free_u32(rt_->raw(), s_);
}

std::vector<uint32_t> DeviceBufferU32::to_host(CudaRuntime& rt) const {
    std::vector<uint32_t> out(s_.len);
    check(forge_memcpy_d2h_u32(rt.raw(), out.data(), s_, s_.len), "to_host_vec");
    return out;
}

// --------------------------------------------------------------- metadata

// metadata.rs:56-67: the next `elements` f32 values' byte range.
void MetadataCursor::reserve(size_t elements, uint64_t* start, uint64_t* end) {
    if ((uint64_t)elements > UINT64_MAX / 4)
        throw Error(FORGE_EINVAL, "parameter byte length overflow");
    const uint64_t bytes = (uint64_t)elements * 4;
    if (position_ > UINT64_MAX - bytes) throw Error(FORGE_EINVAL, "checkpoint offset overflow");
    *start = position_;
    position_ += bytes;
    *end = position_;
}

MatrixMetadata MetadataCursor::matrix(size_t rows, size_t cols) {
    // metadata.rs:30-41.
    if (cols != 0 && rows > SIZE_MAX / cols)
        throw Error(FORGE_EINVAL, "matrix element count overflow");
    MatrixMetadata m;
    m.rows = rows;
    m.cols = cols;
    reserve(rows * cols, &m.byte_start, &m.byte_end);
    return m;
}

VectorMetadata MetadataCursor::vector(size_t len) {
    // metadata.rs:43-50.
    VectorMetadata v;
    v.len = len;
    reserve(len, &v.byte_start, &v.byte_end);
    return v;
}

// ------------------------------------------------------------------ spans

// span.rs:412-416.
static void check_range(size_t buffer_len, size_t offset, size_t len) {
    require(offset <= buffer_len, "device span offset out of bounds");
    require(len <= buffer_len - offset, "device span exceeds its buffer");
}

// span.rs:427-439: [0, len) in chunks of chunk_size, the last one shorter.
static std::vector<forge_slice> split_slices(float* base, size_t len, size_t chunk_size) {
    require(chunk_size > 0, "device span chunk size must be non-zero");
    std::vector<forge_slice> out;
    out.reserve((len + chunk_size - 1) / chunk_size);
    for (size_t off = 0; off < len; off += chunk_size)
        out.push_back(forge_slice{base + off, std::min(chunk_size, len - off)});
    return out;
}

static DeviceBuffer copy_span(CudaRuntime& rt, forge_slice s) {
    DeviceBuffer out = rt.get_uninit_buffer(s.len);
    if (s.len) check(forge_memcpy_d2d(rt.raw(), nullptr, out.slice(), s, s.len), "span to_buffer");
    return out;
}

// A device scalar read back to the host: the reference's reduce_*_buffer
// ends with to_host_vec (span.rs:361-411).
static float scalar_to_host(CudaRuntime& rt, const DeviceBuffer& out) {
    float h = 0.0f;
    check(forge_memcpy_d2h(rt.raw(), &h, out.slice(), 1), "reduce to host");
    return h;
}

DeviceSpan DeviceSpan::from_buffer(const DeviceBuffer& buffer, size_t offset, size_t len) {
    check_range(buffer.len(), offset, len);
    return DeviceSpan(forge_slice{buffer.ptr() + offset, len});
}

std::vector<DeviceSpan> DeviceSpan::chunks(const DeviceBuffer& buffer, size_t chunk_size) {
    std::vector<DeviceSpan> out;
    for (forge_slice s : split_slices(buffer.ptr(), buffer.len(), chunk_size))
        out.push_back(DeviceSpan(s));
    return out;
}

DeviceBuffer DeviceSpan::to_buffer(CudaRuntime& rt) const { return copy_span(rt, s_); }
DeviceBuffer DeviceSpan::to_buffer_async(CudaRuntime& rt) const { return copy_span(rt, s_); }

float DeviceSpan::sum(CudaRuntime& rt) const {
    if (s_.len == 0) return 0.0f;  // span.rs:302-304
    DeviceBuffer out = rt.get_uninit_buffer(1);
    check(forge_reduce_sum(rt.raw(), nullptr, s_, s_.len, out.slice()), "DeviceSpan::sum");
    return scalar_to_host(rt, out);
}

float DeviceSpan::max(CudaRuntime& rt) const {
    if (s_.len == 0) return -3.40282347e38f;  // f32::MIN, span.rs:319-321
    DeviceBuffer out = rt.get_uninit_buffer(1);
    check(forge_reduce_max(rt.raw(), nullptr, s_, s_.len, out.slice()), "DeviceSpan::max");
    return scalar_to_host(rt, out);
}

float DeviceSpan::map_sum(CudaRuntime& rt, MapFn f) const {
    if (s_.len == 0) return 0.0f;  // span.rs:339-341
    DeviceBuffer out = rt.get_uninit_buffer(1);
    check(forge_map_sum(rt.raw(), nullptr, s_, s_.len, f.op, f.p0, out.slice()),
          "DeviceSpan::map_sum");
    return scalar_to_host(rt, out);
}

DeviceSpanMut DeviceSpanMut::from_buffer(DeviceBuffer& buffer, size_t offset, size_t len) {
    check_range(buffer.len(), offset, len);
    return DeviceSpanMut(forge_slice{buffer.ptr() + offset, len});
}

std::vector<DeviceSpanMut> DeviceSpanMut::chunks(DeviceBuffer& buffer, size_t chunk_size) {
    std::vector<DeviceSpanMut> out;
    for (forge_slice s : split_slices(buffer.ptr(), buffer.len(), chunk_size))
        out.push_back(DeviceSpanMut(s));
    return out;
}

DeviceBuffer DeviceSpanMut::to_buffer(CudaRuntime& rt) const { return copy_span(rt, s_); }
DeviceBuffer DeviceSpanMut::to_buffer_async(CudaRuntime& rt) const { return copy_span(rt, s_); }

void DeviceSpanMut::for_each(CudaRuntime& rt, MapFn f) { for_each_on(rt, nullptr, f); }

void DeviceSpanMut::for_each_on(CudaRuntime& rt, const CudaStream* stream, MapFn f) {
    if (s_.len == 0) return;  // span.rs:266-268
    check(forge_map(rt.raw(), stream_raw(stream), s_, s_.len, f.op, f.p0), "for_each");
}

void VectorView::softmax(CudaRuntime& rt) {
    const float m = span_.max(rt);
    span_.for_each(rt, MapFn::exp_shift(m));
    const float total = span_.sum(rt);
    span_.scale(1.0f / total, rt);
}

std::vector<VectorView> Matrix::row_views() {
    std::vector<VectorView> out;
    if (cols_ == 0) return out;
    for (DeviceSpanMut& s : DeviceSpanMut::chunks(buffer_, cols_)) out.push_back(VectorView(s));
    return out;
}

DeviceBuffer CudaRuntime::concat_buffers_from_span(const std::vector<DeviceSpan>& spans) {
    size_t total = 0;
    for (const DeviceSpan& s : spans) total += s.len();
    DeviceBuffer result = get_uninit_buffer(total);
    size_t offset = 0;
    for (const DeviceSpan& s : spans) {
        if (s.len() == 0) continue;
        forge_slice dst{result.ptr() + offset, s.len()};
        check(forge_memcpy_d2d(rt_, nullptr, dst, s.descriptor(), s.len()),
              "concat_buffers_from_span");
        offset += s.len();
    }
    return result;
}

// ---------------------------------------------------------------- runtime

std::unique_ptr<CudaRuntime> CudaRuntime::create(int device, const char* module_path) {
    forge_runtime* rt = nullptr;
    check(forge_runtime_create(device, module_path, &rt), "CudaRuntime::new");
    return std::unique_ptr<CudaRuntime>(new CudaRuntime(rt, true));
}

std::unique_ptr<CudaRuntime> CudaRuntime::borrow(forge_runtime* rt) {
    require(rt != nullptr, "runtime handle is null");
    return std::unique_ptr<CudaRuntime>(new CudaRuntime(rt, false));
}

CudaRuntime::~CudaRuntime() {
    if (!owned_) {
        for (forge_stream* s : streams_) (void)forge_stream_destroy(rt_, s);
        return;
    }
    (void)forge_runtime_destroy(rt_);
}

DeviceBuffer CudaRuntime::get_uninit_buffer(size_t size) {
    forge_slice s;
    check(forge_alloc(rt_, size, &s), "get_uninit_buffer");
    return DeviceBuffer(this, s);
}

DeviceBufferU32 CudaRuntime::get_u32_uninit_buffer(size_t size) {
    forge_slice_u32 s;
    check(forge_alloc_u32(rt_, size, &s), "get_u32_uninit_buffer");
    return DeviceBufferU32(this, s);
}

DeviceBuffer CudaRuntime::get_zerod_buffer(size_t size) {
    forge_slice s;
    check(forge_alloc_zeroed(rt_, size, &s), "get_zerod_buffer");
    return DeviceBuffer(this, s);
}

void CudaRuntime::reserve_buffers(size_t size, size_t count) {
    check(forge_reserve(rt_, size, count), "reserve_buffers");
}

void CudaRuntime::recycle_buffer(DeviceBuffer&& buffer) {
    forge_slice s = buffer.release();
    check(forge_recycle(rt_, s), "recycle_buffer");
}

void CudaRuntime::sync() { check(forge_sync(rt_, nullptr), "sync"); }

std::vector<CudaStream> CudaRuntime::create_extra_streams(size_t count) {
    std::vector<forge_stream*> raw_streams(count);
    check(forge_streams_create(rt_, count, raw_streams.data()), "create_extra_streams");
    std::vector<CudaStream> out;
    for (forge_stream* s : raw_streams) {
        streams_.push_back(s);
        out.emplace_back(s);
    }
    return out;
}

static std::vector<forge_stream*> raws(const std::vector<CudaStream>& streams) {
    std::vector<forge_stream*> r;
    for (const CudaStream& s : streams) r.push_back(s.raw());
    return r;
}

void CudaRuntime::fork_streams(const std::vector<CudaStream>& streams) {
    auto r = raws(streams);
    check(forge_streams_fork(rt_, r.size(), r.data()), "fork_streams");
}

void CudaRuntime::join_streams(const std::vector<CudaStream>& streams) {
    auto r = raws(streams);
    check(forge_streams_join(rt_, r.size(), r.data()), "join_streams");
}

void CudaRuntime::sync_streams(const std::vector<CudaStream>& streams) {
    join_streams(streams);
    sync();
}

void CudaRuntime::stream_join_primary(const CudaStream* waiter) {
    if (waiter) check(forge_stream_wait(rt_, waiter->raw(), nullptr), "CudaStream::join");
}

DeviceBuffer CudaRuntime::concat_buffers(const std::vector<const DeviceBuffer*>& buffers) {
    size_t total = 0;
    for (auto* b : buffers) total += b->len();
    DeviceBuffer result = get_uninit_buffer(total);
    size_t offset = 0;
    for (auto* b : buffers) {
        if (b->len() == 0) continue;
        forge_slice dst{result.ptr() + offset, b->len()};
        check(forge_memcpy_d2d(rt_, nullptr, dst, b->slice(), b->len()), "concat_buffers");
        offset += b->len();
    }
    return result;
}

DeviceBuffer CudaRuntime::span_to_buffer_async(const DeviceSpan& span) {
    return span.to_buffer_async(*this);
}

DeviceBuffer CudaRuntime::clone_buffer(const DeviceBuffer& buffer) {
    DeviceBuffer out = get_uninit_buffer(buffer.len());
    check(forge_memcpy_d2d(rt_, nullptr, out.slice(), buffer.slice(), buffer.len()),
          "clone_buffer");
    return out;
}

void CudaRuntime::gemm_ex(const CudaStream* stream, bool trans_a, bool trans_b, const Matrix& a,
                          const Matrix& b, forge_slice c, size_t m, size_t n, size_t k,
                          const forge_gemm_epilogue& ep) {
    check(forge_gemm_ex_f32(rt_, stream_raw(stream), trans_a ? 1 : 0, trans_b ? 1 : 0, a.slice(),
                            b.slice(), c, m, n, k, &ep),
          "gemm");
}

// ------------------------------------------------------------ matrix.rs

Matrix CudaRuntime::matrix_from_host(const std::vector<float>& values, size_t rows, size_t cols) {
    require(values.size() == rows * cols, "values.len() == rows * cols");
    return matrix_from_host(values.data(), rows, cols);
}

Matrix CudaRuntime::matrix_from_host(const float* values, size_t rows, size_t cols) {
    DeviceBuffer b = get_uninit_buffer(rows * cols);
    check(forge_memcpy_h2d(rt_, b.slice(), values, rows * cols), "matrix_from_host");
    return Matrix(std::move(b), rows, cols);
}

Matrix CudaRuntime::matrix_from_device(forge_slice values, size_t rows, size_t cols) {
    DeviceBuffer b = get_uninit_buffer(rows * cols);
    check(forge_memcpy_d2d(rt_, nullptr, b.slice(), values, rows * cols), "matrix_from_device");
    return Matrix(std::move(b), rows, cols);
}

Matrix CudaRuntime::matrix_multiply(const Matrix& a, const Matrix& b) {
    require(a.cols() == b.rows(), "mat1.cols == mat2.rows");
    Matrix result = new_uninit_matrix(a.rows(), b.cols());
    matrix_multiply_into_on(nullptr, a, b, result);
    return result;
}

Matrix CudaRuntime::matrix_multiply_on(const CudaStream* stream, const Matrix& a,
                                       const Matrix& b) {
    require(a.cols() == b.rows(), "mat1.cols == mat2.rows");
    Matrix result = new_uninit_matrix(a.rows(), b.cols());
    stream_join_primary(stream);
    matrix_multiply_into_on(stream, a, b, result);
    return result;
}

void CudaRuntime::matrix_multiply_into_on(const CudaStream* stream, const Matrix& a,
                                          const Matrix& b, Matrix& result) {
    require(a.cols() == b.rows(), "mat1.cols == mat2.rows");
    require(result.rows() == a.rows() && result.cols() == b.cols(), "result shape");
    check(forge_gemm_f32(rt_, stream_raw(stream), a.slice(), b.slice(), result.slice(), a.rows(),
                         b.cols(), a.cols()),
          "matrix_multiply");
}

Matrix CudaRuntime::matrix_add(const Matrix& a, const Matrix& b) {
    return matrix_binary(a, b, BinaryOp::Add);
}
Matrix CudaRuntime::matrix_sub(const Matrix& a, const Matrix& b) {
    return matrix_binary(a, b, BinaryOp::Sub);
}
Matrix CudaRuntime::matrix_mul(const Matrix& a, const Matrix& b) {
    return matrix_binary(a, b, BinaryOp::Mul);
}
Matrix CudaRuntime::matrix_div(const Matrix& a, const Matrix& b) {
    return matrix_binary(a, b, BinaryOp::Div);
}

Matrix CudaRuntime::matrix_binary(const Matrix& a, const Matrix& b, BinaryOp op) {
    return matrix_binary_on(nullptr, a, b, op);
}

Matrix CudaRuntime::matrix_binary_on(const CudaStream* stream, const Matrix& a, const Matrix& b,
                                     BinaryOp op) {
    require(a.rows() == b.rows() && a.cols() == b.cols(), "matrix_binary shapes");
    Matrix out = new_uninit_matrix(a.rows(), a.cols());
    stream_join_primary(stream);
    check(forge_binary(rt_, stream_raw(stream), a.slice(), b.slice(), out.slice(), a.rows() * a.cols(),
                       (forge_binary_op)op),
          "matrix_binary");
    return out;
}

void CudaRuntime::recycle_matrix(Matrix&& m) { recycle_buffer(m.into_buffer()); }

Matrix CudaRuntime::new_matrix(InitType init, size_t rows, size_t cols) {
    size_t size = rows * cols;
    if (init == InitType::Zero) return Matrix(get_zerod_buffer(size), rows, cols);
    DeviceBuffer b = get_uninit_buffer(size);
    switch (init) {
    case InitType::Sequence:
        check(forge_fill_seq(rt_, nullptr, b.slice(), size, 1), "new_matrix");
        break;
    case InitType::Reserve:
        check(forge_fill_seq(rt_, nullptr, b.slice(), size, 0), "new_matrix");
        break;
    case InitType::Random: {
        // rand::random() seed (matrix.rs:284): non-deterministic by design.
        std::random_device rd;
        check(forge_fill_random(rt_, nullptr, b.slice(), size, rd()), "new_matrix");
        break;
    }
    case InitType::Zero: break;
    }
    return Matrix(std::move(b), rows, cols);
}

Matrix CudaRuntime::new_uninit_matrix(size_t rows, size_t cols) {
    return Matrix(get_uninit_buffer(rows * cols), rows, cols);
}

Matrix CudaRuntime::clone_matrix(const Matrix& m) {
    return Matrix(clone_buffer(m.buffer()), m.rows(), m.cols());
}

Matrix CudaRuntime::clone_matrix_on(const Matrix& m, const CudaStream* stream) {
    DeviceBuffer b = get_uninit_buffer(m.len());
    stream_join_primary(stream);
    check(forge_memcpy_d2d(rt_, stream_raw(stream), b.slice(), m.slice(), m.len()), "clone_matrix_on");
    return Matrix(std::move(b), m.rows(), m.cols());
}

// -------------------------------------------------------------- norm.rs

Matrix CudaRuntime::softmax_rows_backward(const Matrix& p, const Matrix& g) {
    require(p.rows() == g.rows() && p.cols() == g.cols(), "softmax_rows_backward shapes");
    Matrix out = new_uninit_matrix(p.rows(), p.cols());
    check(forge_softmax_rows_bwd(rt_, nullptr, p.slice(), g.slice(), out.slice(), p.rows(),
                                 p.cols()),
          "softmax_rows_backward");
    return out;
}

static forge_slice opt_slice(const Vector* v) { return v ? v->slice() : forge_slice{nullptr, 0}; }

Matrix CudaRuntime::layer_norm_backward(const Matrix& x, const Matrix& g, const Vector* gamma,
                                        Vector* dgamma, Vector* dbeta) {
    require(x.rows() == g.rows() && x.cols() == g.cols(), "layer_norm_backward shapes");
    Matrix out = new_uninit_matrix(x.rows(), x.cols());
    check(forge_layer_norm_bwd(rt_, nullptr, x.slice(), g.slice(), opt_slice(gamma), out.slice(),
                               opt_slice(dgamma), opt_slice(dbeta), x.rows(), x.cols(), 1e-5f),
          "layer_norm_backward");
    return out;
}

Matrix CudaRuntime::rms_norm_backward(const Matrix& x, const Matrix& g, const Vector* gamma,
                                      Vector* dgamma) {
    require(x.rows() == g.rows() && x.cols() == g.cols(), "rms_norm_backward shapes");
    Matrix out = new_uninit_matrix(x.rows(), x.cols());
    check(forge_rms_norm_bwd(rt_, nullptr, x.slice(), g.slice(), opt_slice(gamma), out.slice(),
                             opt_slice(dgamma), x.rows(), x.cols(), 1e-5f),
          "rms_norm_backward");
    return out;
}

// -------------------------------------------------------------- rows.rs

Vector CudaRuntime::matrix_sum_rows(const Matrix& m) { return matrix_sum_rows_on(m, nullptr); }

Vector CudaRuntime::matrix_sum_rows_on(const Matrix& m, const CudaStream* stream) {
    DeviceBuffer b = get_uninit_buffer(m.rows());
    stream_join_primary(stream);
    check(forge_sum_rows(rt_, stream_raw(stream), m.slice(), b.slice(), m.rows(), m.cols()),
          "matrix_sum_rows");
    return Vector(std::move(b));
}

Vector CudaRuntime::matrix_sum_cols(const Matrix& m, const CudaStream* stream) {
    DeviceBuffer b = get_uninit_buffer(m.cols());
    stream_join_primary(stream);
    check(forge_sum_cols(rt_, stream_raw(stream), m.slice(), b.slice(), m.rows(), m.cols()),
          "matrix_sum_cols");
    return Vector(std::move(b));
}

// ----------------------------------------------------------- convert.rs

Matrix CudaRuntime::matrix_transpose(const Matrix& m) { return matrix_transpose_on(m, nullptr); }

Matrix CudaRuntime::matrix_transpose_on(const Matrix& m, const CudaStream* stream) {
    Matrix out = new_uninit_matrix(m.cols(), m.rows());
    stream_join_primary(stream);
    check(forge_transpose_f32(rt_, stream_raw(stream), m.slice(), out.slice(), m.rows(), m.cols()),
          "matrix_transpose");
    return out;
}

Matrix CudaRuntime::vector_zip(const std::vector<Vector>& vecs) {
    require(!vecs.empty(), "vector_zip of no vectors");
    std::vector<const DeviceBuffer*> bufs;
    for (const Vector& v : vecs) {
        require(v.len() == vecs[0].len(), "vector_zip lengths");
        bufs.push_back(&v.buffer());
    }
    return Matrix(concat_buffers(bufs), vecs.size(), vecs[0].len());
}

std::vector<Vector> CudaRuntime::matrix_split(const Matrix& m) {
    std::vector<Vector> out;
    for (size_t r = 0; r < m.rows(); r++) {
        DeviceBuffer b = get_uninit_buffer(m.cols());
        forge_slice src{m.slice().ptr + r * m.cols(), m.cols()};
        check(forge_memcpy_d2d(rt_, nullptr, b.slice(), src, m.cols()), "matrix_split");
        out.emplace_back(std::move(b));
    }
    return out;
}

Matrix CudaRuntime::broadcast(const Vector& v, size_t copies) {
    std::vector<const DeviceBuffer*> bufs(copies, &v.buffer());
    return Matrix(concat_buffers(bufs), copies, v.len());
}

Vector CudaRuntime::extract_vector(Matrix&& m) {
    require(m.rows() > 0, "cannot extract a vector from an empty matrix");
    if (m.rows() == 1) return Vector(m.into_buffer());
    DeviceBuffer b = get_uninit_buffer(m.cols());
    check(forge_memcpy_d2d(rt_, nullptr, b.slice(), m.slice(), m.cols()), "extract_vector");
    return Vector(std::move(b));
}

std::vector<Matrix> CudaRuntime::matrix_slice(const Matrix& m, size_t cols, size_t rows) {
    require(cols > 0 && rows > 0, "matrix slice dims must be non-zero");
    require(m.cols() % cols == 0 && m.rows() % rows == 0, "matrix slice divisibility");
    std::vector<Matrix> out;
    for (size_t tr = 0; tr < m.rows() / rows; tr++) {
        for (size_t tc = 0; tc < m.cols() / cols; tc++) {
            DeviceBuffer b = get_uninit_buffer(rows * cols);
            for (size_t r = 0; r < rows; r++) {
                forge_slice src{m.slice().ptr + (tr * rows + r) * m.cols() + tc * cols, cols};
                forge_slice dst{b.ptr() + r * cols, cols};
                check(forge_memcpy_d2d(rt_, nullptr, dst, src, cols), "matrix_slice");
            }
            out.emplace_back(std::move(b), rows, cols);
        }
    }
    return out;
}

Vector CudaRuntime::matrix_into_vector(Matrix&& m) { return Vector(m.into_buffer()); }

Matrix CudaRuntime::vector_into_matrix(Vector&& v) {
    size_t n = v.len();
    return Matrix(std::move(v.buffer()), n, 1);
}

// ---------------------------------------------------- vector_runtime.rs

Vector CudaRuntime::vector_from_host(const std::vector<float>& values) {
    return vector_from_host(values.data(), values.size());
}

Vector CudaRuntime::vector_from_host(const float* values, size_t n) {
    DeviceBuffer b = get_uninit_buffer(n);
    check(forge_memcpy_h2d(rt_, b.slice(), values, n), "vector_from_host");
    return Vector(std::move(b));
}

Vector CudaRuntime::vector_from_device(forge_slice values) {
    DeviceBuffer b = get_uninit_buffer(values.len);
    check(forge_memcpy_d2d(rt_, nullptr, b.slice(), values, values.len), "vector_from_device");
    return Vector(std::move(b));
}

void CudaRuntime::recycle_vector(Vector&& v) { recycle_buffer(std::move(v.buffer())); }

Vector CudaRuntime::new_vector(InitType init, size_t size) {
    Matrix m = new_matrix(init, 1, size);
    return Vector(m.into_buffer());
}

Vector CudaRuntime::clone_vector(const Vector& v) { return Vector(clone_buffer(v.buffer())); }

Vector CudaRuntime::clone_vector_on(const Vector& v, const CudaStream* stream) {
    DeviceBuffer b = get_uninit_buffer(v.len());
    stream_join_primary(stream);
    check(forge_memcpy_d2d(rt_, stream_raw(stream), b.slice(), v.slice(), v.len()), "clone_vector_on");
    return Vector(std::move(b));
}

Vector CudaRuntime::vector_add(const Vector& a, const Vector& b) {
    return vector_binary(a, b, BinaryOp::Add);
}
Vector CudaRuntime::vector_sub(const Vector& a, const Vector& b) {
    return vector_binary(a, b, BinaryOp::Sub);
}
Vector CudaRuntime::vector_mul(const Vector& a, const Vector& b) {
    return vector_binary(a, b, BinaryOp::Mul);
}
Vector CudaRuntime::vector_div(const Vector& a, const Vector& b) {
    return vector_binary(a, b, BinaryOp::Div);
}

Vector CudaRuntime::vector_binary(const Vector& a, const Vector& b, BinaryOp op) {
    require(a.len() == b.len(), "vector_binary lengths");
    DeviceBuffer out = get_uninit_buffer(a.len());
    check(forge_binary(rt_, nullptr, a.slice(), b.slice(), out.slice(), a.len(),
                       (forge_binary_op)op),
          "vector_binary");
    return Vector(std::move(out));
}

// ----------------------------------------------------------------- Vector

std::vector<float> Vector::to_host(CudaRuntime& rt) const {
    std::vector<float> out(len());
    check(forge_memcpy_d2h(rt.raw(), out.data(), slice(), len()), "Vector::to_host");
    return out;
}

void Vector::add_scalar(float value, CudaRuntime& rt) {
    check(forge_map(rt.raw(), nullptr, slice(), len(), FORGE_MAP_ADD, value), "add_scalar");
}

void Vector::scale(float value, CudaRuntime& rt) { scale_on(value, rt, nullptr); }

void Vector::scale_on(float value, CudaRuntime& rt, const CudaStream* stream) {
    check(forge_map(rt.raw(), stream_raw(stream), slice(), len(), FORGE_MAP_SCALE, value), "scale");
}

static float reduce_to_host(CudaRuntime& rt, const Vector& v, bool is_max) {
    if (v.len() == 0) return is_max ? -3.40282347e38f : 0.0f;  // span.rs:302-321
    DeviceBuffer out = rt.get_uninit_buffer(1);
    if (is_max)
        check(forge_reduce_max(rt.raw(), nullptr, v.slice(), v.len(), out.slice()), "max");
    else
        check(forge_reduce_sum(rt.raw(), nullptr, v.slice(), v.len(), out.slice()), "sum");
    float h = 0.0f;
    check(forge_memcpy_d2h(rt.raw(), &h, out.slice(), 1), "reduce to host");
    return h;
}

float Vector::sum(CudaRuntime& rt) const { return reduce_to_host(rt, *this, false); }
float Vector::max(CudaRuntime& rt) const { return reduce_to_host(rt, *this, true); }

void Vector::exp_shifted(float offset, CudaRuntime& rt) {
    check(forge_map(rt.raw(), nullptr, slice(), len(), FORGE_MAP_EXP_SHIFT, offset),
          "exp_shifted");
}

void Vector::softmax(CudaRuntime& rt) {
    // vector.rs:53-58: max, exp(x - max), sum, scale by 1/sum.
    float m = max(rt);
    exp_shifted(m, rt);
    float s = sum(rt);
    scale(1.0f / s, rt);
}

void Vector::binary_assign(const Vector& rhs, BinaryOp op, CudaRuntime& rt) {
    binary_assign_on(rhs, op, rt, nullptr);
}

void Vector::binary_assign_on(const Vector& rhs, BinaryOp op, CudaRuntime& rt,
                              const CudaStream* stream) {
    require(len() == rhs.len(), "Vector::binary_assign lengths");
    check(forge_binary_assign(rt.raw(), stream_raw(stream), slice(), rhs.slice(), len(),
                              (forge_binary_op)op),
          "Vector::binary_assign");
}

float Vector::dot(const Vector& rhs, CudaRuntime& rt) const {
    require(len() == rhs.len(), "dot lengths");
    Vector product = rt.vector_mul(*this, rhs);
    return product.sum(rt);
}

bool Vector::equals(const Vector& rhs, CudaRuntime& rt) const {
    // vector.rs:117-136: the comparison into a one-element u32 buffer.
    require(len() == rhs.len(), "equals lengths");
    DeviceBufferU32 result = rt.get_u32_uninit_buffer(1);
    check(forge_compare_u32(rt.raw(), nullptr, slice(), rhs.slice(), len(), result.slice()),
          "equals");
    return result.to_host(rt)[0] == 0;
}

// ----------------------------------------------------------------- Matrix

std::vector<float> Matrix::to_host(CudaRuntime& rt) const {
    std::vector<float> out(len());
    check(forge_memcpy_d2h(rt.raw(), out.data(), slice(), len()), "Matrix::to_host");
    return out;
}

void Matrix::scale(float value, CudaRuntime& rt) { map(FORGE_MAP_SCALE, value, rt); }
void Matrix::add_scalar(float value, CudaRuntime& rt) { map(FORGE_MAP_ADD, value, rt); }

void Matrix::map(forge_map_op op, float p0, CudaRuntime& rt, const CudaStream* stream) {
    if (len() == 0) return;
    check(forge_map(rt.raw(), stream_raw(stream), slice(), len(), op, p0), "Matrix::for_each");
}

void Matrix::binary_assign(const Matrix& rhs, BinaryOp op, CudaRuntime& rt) {
    binary_assign_on(rhs, op, rt, nullptr);
}

void Matrix::binary_assign_on(const Matrix& rhs, BinaryOp op, CudaRuntime& rt,
                              const CudaStream* stream) {
    require(rows_ == rhs.rows_ && cols_ == rhs.cols_, "binary_assign shapes");
    check(forge_binary_assign(rt.raw(), stream_raw(stream), slice(), rhs.slice(), len(),
                              (forge_binary_op)op),
          "Matrix::binary_assign");
}

void Matrix::causal_mask(CudaRuntime& rt) {
    if (rows_ == 0) return;
    check(forge_causal_mask(rt.raw(), nullptr, slice(), rows_, cols_), "causal_mask");
}

void Matrix::softmax_rows(CudaRuntime& rt) {
    if (rows_ == 0) return;
    check(forge_softmax_rows(rt.raw(), nullptr, slice(), rows_, cols_), "softmax_rows");
}

void Matrix::layer_norm(CudaRuntime& rt, const Vector* gamma, const Vector* beta) {
    if (rows_ == 0) return;
    check(forge_layer_norm_rows(rt.raw(), nullptr, slice(), opt_slice(gamma), opt_slice(beta),
                                rows_, cols_, 1e-5f),
          "layer_norm");
}

void Matrix::rms_norm(CudaRuntime& rt, const Vector* gamma) {
    if (rows_ == 0) return;
    check(forge_rms_norm_rows(rt.raw(), nullptr, slice(), opt_slice(gamma), rows_, cols_, 1e-5f),
          "rms_norm");
}

void Matrix::binary_assign_by_rows(const Vector& vec, BinaryOp op, CudaRuntime& rt) {
    binary_assign_by_rows_on(vec, op, rt, nullptr);
}

void Matrix::binary_assign_by_rows_on(const Vector& vec, BinaryOp op, CudaRuntime& rt,
                                      const CudaStream* stream) {
    require(cols_ == vec.len(), "binary_assign_by_rows: cols == vec.len()");
    if (len() == 0) return;
    check(forge_binary_assign_by_rows(rt.raw(), stream_raw(stream), slice(), vec.slice(), rows_, cols_,
                                      (forge_binary_op)op),
          "binary_assign_by_rows");
}

}  // namespace oxforge
