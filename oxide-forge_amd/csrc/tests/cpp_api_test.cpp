// cpp_api_test.cpp -- exercises the C++ drop-in API of include/oxforge_net.hpp
// (CudaRuntime / Matrix / Vector / streams / pool / conversions / Linear /
// MLP) on a GPU against host arithmetic written out here.  Built in-tree by
// the Makefile as lib/oxforge_cpp_api_test; run by tests/test_gpu_cpp_api.py.
// Exit status 0 when every check passes; one line per check group.
//
// Bars: bit-exact for copies, fills, transposes, conversions, single
// rounded elementwise ops and integer-valued sums; 1e-4 relative-to-max for
// the GEMM; 1e-5 absolute for softmax and the norms.
#include "oxforge_checkpoint.hpp"
#include "oxforge_net.hpp"

#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

using namespace oxforge;

static int g_failures = 0;

#define CHECK(cond, what)                                                   \
    do {                                                                    \
        if (!(cond)) {                                                      \
            std::printf("FAIL %s (%s:%d)\n", what, __FILE__, __LINE__);     \
            g_failures++;                                                   \
        }                                                                   \
    } while (0)

static std::vector<float> iota(size_t n, float scale = 1.0f, float offset = 0.0f) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; i++) v[i] = offset + scale * (float)((i * 7919u) % 97u);
    return v;
}

static std::vector<float> uniform(size_t n, uint64_t seed) {
    std::vector<float> v(n);
    uint64_t x = seed * 0x9E3779B97F4A7C15ull + 1;
    for (size_t i = 0; i < n; i++) {
        x ^= x >> 12;
        x ^= x << 25;
        x ^= x >> 27;
        v[i] = (float)((double)((x * 0x2545F4914F6CDD1Dull) >> 40) / (double)(1ull << 24)) * 2.0f - 1.0f;
    }
    return v;
}

static double max_abs(const std::vector<double>& v) {
    double m = 0;
    for (double x : v) m = std::fmax(m, std::fabs(x));
    return m;
}

static void group(const char* name, int before) {
    std::printf("%s %s\n", g_failures == before ? "PASS" : "FAIL", name);
}

// The span group's inputs and results, for the oracle comparison of
// tests/test_gpu_cpp_api.py (written when a dump directory is given).
static void dump(const std::string& path, const std::vector<float>& v) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) {
        std::printf("FAIL cannot write %s\n", path.c_str());
        g_failures++;
        return;
    }
    std::fwrite(v.data(), sizeof(float), v.size(), f);
    std::fclose(f);
}

// ------------------------------------------------ metadata as JSON
// get_meta_data results in the field names and nesting of the reference's
// serde structs (the form oracle/checkpoint.py builds), for the comparison
// of tests/test_gpu_cpp_api.py.  Absent options are left out, as serde's
// skip of None in the checkpoint writer.
static const char* act_name(Activation a) {
    switch (a) {
    case Activation::Gelu: return "gelu";
    case Activation::Relu: return "relu";
    case Activation::Silu: return "silu";
    default: return "identity";
    }
}

static std::string json(const MatrixMetadata& m) {
    return "{\"rows\": " + std::to_string(m.rows) + ", \"cols\": " + std::to_string(m.cols) +
           ", \"byte_start\": " + std::to_string(m.byte_start) +
           ", \"byte_end\": " + std::to_string(m.byte_end) + "}";
}

static std::string json(const VectorMetadata& v) {
    return "{\"len\": " + std::to_string(v.len) + ", \"byte_start\": " +
           std::to_string(v.byte_start) + ", \"byte_end\": " + std::to_string(v.byte_end) + "}";
}

static std::string json(const LinearMetadata& l) {
    std::string s = "{\"input_neurons\": " + std::to_string(l.input_neurons) +
                    ", \"output_neurons\": " + std::to_string(l.output_neurons) +
                    ", \"activation\": \"" + act_name(l.activation) + "\", \"weights\": " +
                    json(l.weights);
    if (l.bias) s += ", \"bias\": " + json(*l.bias);
    return s + "}";
}

static std::string json(const MlpMetadata& m) {
    std::string s = "{\"layer_count\": " + std::to_string(m.layer_count) +
                    ", \"loss\": \"mean_squared_error\"";
    if (m.residual)
        s += ", \"residual\": {\"start\": " + std::to_string(m.residual->start) +
             ", \"end\": " + std::to_string(m.residual->end) + "}";
    s += ", \"layers\": [";
    for (size_t i = 0; i < m.layers.size(); i++) s += (i ? ", " : "") + json(m.layers[i]);
    return s + "]}";
}

static std::string json(const TransformerMetadata& t) {
    std::string s = "{\"block_count\": " + std::to_string(t.block_count) +
                    ", \"attention_residual\": " + (t.attention_residual ? "true" : "false") +
                    ", \"feed_forward_residual\": " +
                    (t.feed_forward_residual ? "true" : "false") + ", \"normalization\": \"" +
                    (t.normalization == NormType::Rms ? "rms" : "layer") +
                    "\", \"position\": " + json(t.position) + ", \"query\": " + json(t.query) +
                    ", \"key\": " + json(t.key) + ", \"value\": " + json(t.value) +
                    ", \"feed_forward\": " + json(t.feed_forward) +
                    ", \"output\": " + json(t.output);
    const std::pair<const char*, const std::optional<VectorMetadata>*> norms[] = {
        {"norm1_gamma", &t.norm1_gamma}, {"norm1_beta", &t.norm1_beta},
        {"norm2_gamma", &t.norm2_gamma}, {"norm2_beta", &t.norm2_beta}};
    for (const auto& n : norms)
        if (*n.second) s += std::string(", \"") + n.first + "\": " + json(**n.second);
    return s + "}";
}

// Writes <dir>/<name>.json ({"meta": ..., "data_bytes": N}) and
// <dir>/<name>.f32 (every get_data block back to back).
static void write_model(const std::string& dir, const std::string& name, const std::string& meta,
                        uint64_t data_bytes, const std::vector<HostData>& data) {
    FILE* f = std::fopen((dir + "/" + name + ".json").c_str(), "w");
    if (!f) {
        std::printf("FAIL cannot write %s.json\n", name.c_str());
        g_failures++;
        return;
    }
    std::fprintf(f, "{\"meta\": %s, \"data_bytes\": %llu}\n", meta.c_str(),
                 (unsigned long long)data_bytes);
    std::fclose(f);
    std::vector<float> all;
    for (const HostData& d : data) all.insert(all.end(), d.values().begin(), d.values().end());
    dump(dir + "/" + name + ".f32", all);
}

template <typename M>
static void describe(const std::string& dir, const std::string& name, const M& model,
                     CudaRuntime& R) {
    MetadataCursor cursor;
    auto meta = model.get_meta_data(cursor);
    write_model(dir, name, json(meta), cursor.data_bytes(), model.get_data(R));
}

// --metadata <dir>: loads the checkpoints that tests/test_gpu_cpp_api.py wrote
// into <dir> with the reference-format writer of the oracle (linear,
// linear_nobias, mlp, transformer_rms, transformer_layer) into every model
// type that can hold them and writes what get_meta_data / get_data return.
static int metadata_mode(const std::string& dir, CudaRuntime& R) {
    namespace ck = checkpoint;
    for (const char* name : {"linear", "linear_nobias"}) {
        Linear l = ck::load_linear(dir + "/" + name, R);
        describe(dir, std::string(name) + ".Linear", l, R);
    }
    {
        MlpExecutor e = ck::load_mlp(dir + "/mlp", R);
        describe(dir, "mlp.MlpExecutor", e, R);
        InferenceMLP i = ck::load_inference_mlp(dir + "/mlp", R);
        describe(dir, "mlp.InferenceMLP", i, R);
        TrainingMlp t = ck::load_training_mlp(dir + "/mlp", R);
        describe(dir, "mlp.TrainingMlp", t, R);
    }
    for (const char* name : {"transformer_rms", "transformer_layer"}) {
        const std::string path = dir + "/" + name;
        encoder::InferenceTransformer e = ck::load_transformer(path, R);
        describe(dir, std::string(name) + ".encoder.InferenceTransformer", e, R);
        encoder::TrainingTransformer t = ck::load_training_transformer(path, R);
        describe(dir, std::string(name) + ".encoder.TrainingTransformer", t, R);
        decoder::InferenceTransformer d = ck::load_decoder_transformer(path, R);
        describe(dir, std::string(name) + ".decoder.InferenceTransformer", d, R);
    }
    R.sync();
    std::printf("%s: %d failed check(s)\n", g_failures ? "FAILED" : "OK", g_failures);
    return g_failures ? 1 : 0;
}

int main(int argc, char** argv) {
    if (argc > 2 && std::string(argv[1]) == "--metadata") {
        int ndev = 0;
        if (forge_device_count(&ndev) != FORGE_OK || ndev == 0) {
            std::printf("no GPU\n");
            return 2;
        }
        auto rt = CudaRuntime::create();
        return metadata_mode(argv[2], *rt);
    }
    const std::string dump_dir = argc > 1 ? argv[1] : "";
    int dev = 0;
    if (forge_device_count(&dev) != FORGE_OK || dev == 0) {
        std::printf("no GPU\n");
        return 2;
    }
    auto rt = CudaRuntime::create();
    CudaRuntime& R = *rt;

    // ---------------------------------------------------- host round trip
    {
        int f = g_failures;
        auto h = uniform(37 * 19, 1);
        Matrix m = R.matrix_from_host(h, 37, 19);
        CHECK(m.rows() == 37 && m.cols() == 19 && m.len() == h.size(), "matrix shape");
        CHECK(m.to_host(R) == h, "matrix round trip");
        Vector v = R.vector_from_host(h);
        CHECK(v.len() == h.size() && v.to_host(R) == h, "vector round trip");
        group("round_trip", f);
    }

    // ----------------------------------------------------------- init types
    {
        int f = g_failures;
        Vector seq = R.new_vector(InitType::Sequence, 1000);
        Vector rev = R.new_vector(InitType::Reserve, 1000);
        Vector zero = R.new_vector(InitType::Zero, 1000);
        Vector rnd = R.new_vector(InitType::Random, 1000);
        auto s = seq.to_host(R), r = rev.to_host(R), z = zero.to_host(R), q = rnd.to_host(R);
        bool ok_s = true, ok_r = true, ok_z = true, ok_q = true;
        for (size_t i = 0; i < 1000; i++) {
            ok_s = ok_s && s[i] == (float)i;             // elementwise.rs:23-34 ascending
            ok_r = ok_r && r[i] == (float)(1000 - i);    // descending: len - index
            ok_z = ok_z && z[i] == 0.0f;
            ok_q = ok_q && q[i] >= 0.0f && q[i] <= 1.0f;  // hash / u32::MAX
        }
        CHECK(ok_s, "InitType::Sequence");
        CHECK(ok_r, "InitType::Reserve");
        CHECK(ok_z, "InitType::Zero");
        CHECK(ok_q, "InitType::Random range");
        Matrix ms = R.new_matrix(InitType::Sequence, 4, 5);
        auto mh = ms.to_host(R);
        CHECK(ms.rows() == 4 && ms.cols() == 5 && mh[19] == 19.0f, "new_matrix Sequence");
        group("init_types", f);
    }

    // ------------------------------------------------------------------ GEMM
    {
        int f = g_failures;
        const size_t M = 70, K = 45, N = 33;
        auto a = uniform(M * K, 2), b = uniform(K * N, 3);
        Matrix A = R.matrix_from_host(a, M, K), B = R.matrix_from_host(b, K, N);
        Matrix C = R.matrix_multiply(A, B);
        auto c = C.to_host(R);
        std::vector<double> ref(M * N, 0.0), err(M * N);
        for (size_t i = 0; i < M; i++)
            for (size_t k = 0; k < K; k++)
                for (size_t j = 0; j < N; j++) ref[i * N + j] += (double)a[i * K + k] * b[k * N + j];
        for (size_t i = 0; i < M * N; i++) err[i] = c[i] - ref[i];
        CHECK(C.rows() == M && C.cols() == N, "matrix_multiply shape");
        CHECK(max_abs(err) <= 1e-4 * max_abs(ref), "matrix_multiply vs f64");
        // On an extra stream, forked from and joined to the primary.
        auto streams = R.create_extra_streams(1);
        Matrix C2 = R.matrix_multiply_on(&streams[0], A, B);
        R.join_streams(streams);
        CHECK(C2.to_host(R) == c, "matrix_multiply_on a forked stream");
        group("gemm", f);
    }

    // ------------------------------------------------ elementwise, bit-exact
    {
        int f = g_failures;
        const size_t rows = 13, cols = 21, n = rows * cols;
        auto x = uniform(n, 4), y = uniform(n, 5);
        for (auto& v : y) v = v == 0.0f ? 0.5f : v;
        Matrix X = R.matrix_from_host(x, rows, cols), Y = R.matrix_from_host(y, rows, cols);
        const BinaryOp ops[4] = {BinaryOp::Add, BinaryOp::Sub, BinaryOp::Mul, BinaryOp::Div};
        for (BinaryOp op : ops) {
            auto got = R.matrix_binary(X, Y, op).to_host(R);
            bool ok = true;
            for (size_t i = 0; i < n; i++) {
                float want = op == BinaryOp::Add ? x[i] + y[i]
                             : op == BinaryOp::Sub ? x[i] - y[i]
                             : op == BinaryOp::Mul ? x[i] * y[i]
                                                   : x[i] / y[i];
                ok = ok && got[i] == want;
            }
            CHECK(ok, "matrix_binary");
        }
        Matrix S = R.clone_matrix(X);
        S.scale(0.37f, R);
        S.add_scalar(-1.5f, R);
        auto sh = S.to_host(R);
        bool ok = true;
        for (size_t i = 0; i < n; i++) ok = ok && sh[i] == x[i] * 0.37f + -1.5f;
        CHECK(ok, "scale + add_scalar");
        CHECK(X.to_host(R) == x, "clone_matrix leaves the source");
        Matrix T = R.clone_matrix(X);
        T.binary_assign(Y, BinaryOp::Mul, R);
        auto th = T.to_host(R);
        ok = true;
        for (size_t i = 0; i < n; i++) ok = ok && th[i] == x[i] * y[i];
        CHECK(ok, "binary_assign");
        auto rv = uniform(cols, 6);
        Vector row = R.vector_from_host(rv);
        Matrix Bc = R.clone_matrix(X);
        Bc.binary_assign_by_rows(row, BinaryOp::Sub, R);
        auto bh = Bc.to_host(R);
        ok = true;
        for (size_t i = 0; i < n; i++) ok = ok && bh[i] == x[i] - rv[i % cols];
        CHECK(ok, "binary_assign_by_rows");
        group("elementwise", f);
    }

    // --------------------------------------------------- rows: softmax, norms
    {
        int f = g_failures;
        const size_t rows = 9, cols = 37;
        auto x = uniform(rows * cols, 7), g = uniform(rows * cols, 8);
        for (auto& v : x) v *= 3.0f;
        std::vector<double> sm(rows * cols), ln(rows * cols), rms(rows * cols);
        for (size_t r = 0; r < rows; r++) {
            const float* xr = &x[r * cols];
            double m = -1e300, s = 0, mean = 0, var = 0, q = 0;
            for (size_t c = 0; c < cols; c++) m = std::fmax(m, xr[c]);
            for (size_t c = 0; c < cols; c++) s += std::exp(xr[c] - m);
            for (size_t c = 0; c < cols; c++) mean += xr[c];
            mean /= cols;
            for (size_t c = 0; c < cols; c++) var += (xr[c] - mean) * (xr[c] - mean);
            var /= cols;
            for (size_t c = 0; c < cols; c++) q += (double)xr[c] * xr[c];
            for (size_t c = 0; c < cols; c++) {
                sm[r * cols + c] = std::exp(xr[c] - m) / s;
                ln[r * cols + c] = (xr[c] - mean) / std::sqrt(var + 1e-5);
                rms[r * cols + c] = xr[c] / std::sqrt(q / cols + 1e-5);
            }
        }
        auto close = [&](const std::vector<float>& a, const std::vector<double>& b) {
            double e = 0;
            for (size_t i = 0; i < a.size(); i++) e = std::fmax(e, std::fabs(a[i] - b[i]));
            return e <= 1e-5;
        };
        Matrix P = R.matrix_from_host(x, rows, cols);
        P.softmax_rows(R);
        CHECK(close(P.to_host(R), sm), "softmax_rows");
        Matrix L = R.matrix_from_host(x, rows, cols);
        L.layer_norm(R);
        CHECK(close(L.to_host(R), ln), "layer_norm");
        Matrix Q = R.matrix_from_host(x, rows, cols);
        Q.rms_norm(R);
        CHECK(close(Q.to_host(R), rms), "rms_norm");
        // Backward: softmax dx = p (g - sum p g); LN / RMS vs host f64.
        Matrix G = R.matrix_from_host(g, rows, cols);
        auto dsm = R.softmax_rows_backward(P, G).to_host(R);
        auto ph = P.to_host(R);
        std::vector<double> dref(rows * cols);
        for (size_t r = 0; r < rows; r++) {
            double s = 0;
            for (size_t c = 0; c < cols; c++) s += (double)ph[r * cols + c] * g[r * cols + c];
            for (size_t c = 0; c < cols; c++)
                dref[r * cols + c] = ph[r * cols + c] * (g[r * cols + c] - s);
        }
        CHECK(close(dsm, dref), "softmax_rows_backward");
        Matrix Xm = R.matrix_from_host(x, rows, cols);
        auto dln = R.layer_norm_backward(Xm, G).to_host(R);
        for (size_t r = 0; r < rows; r++) {
            const float* xr = &x[r * cols];
            const float* gr = &g[r * cols];
            double mean = 0, var = 0, A = 0, Bs = 0;
            for (size_t c = 0; c < cols; c++) mean += xr[c];
            mean /= cols;
            for (size_t c = 0; c < cols; c++) var += (xr[c] - mean) * (xr[c] - mean);
            var /= cols;
            const double rs = 1.0 / std::sqrt(var + 1e-5);
            for (size_t c = 0; c < cols; c++) {
                A += gr[c];
                Bs += gr[c] * (xr[c] - mean) * rs;
            }
            for (size_t c = 0; c < cols; c++)
                dref[r * cols + c] = rs / cols * (cols * gr[c] - A - (xr[c] - mean) * rs * Bs);
        }
        CHECK(close(dln, dref), "layer_norm_backward");
        auto drms = R.rms_norm_backward(Xm, G).to_host(R);
        for (size_t r = 0; r < rows; r++) {
            const float* xr = &x[r * cols];
            const float* gr = &g[r * cols];
            double q = 0, d = 0;
            for (size_t c = 0; c < cols; c++) {
                q += (double)xr[c] * xr[c];
                d += (double)xr[c] * gr[c];
            }
            const double inv = 1.0 / std::sqrt(q / cols + 1e-5);
            for (size_t c = 0; c < cols; c++)
                dref[r * cols + c] = gr[c] * inv - xr[c] * (d / cols * inv * inv * inv);
        }
        CHECK(close(drms, dref), "rms_norm_backward");
        // Causal mask then softmax: masked entries are exactly zero and each
        // row sums to one over its unmasked prefix.
        std::vector<float> sq(x.begin(), x.begin() + rows * rows);
        Matrix Cm = R.matrix_from_host(sq, rows, rows);
        Cm.causal_mask(R);
        Cm.softmax_rows(R);
        auto ch = Cm.to_host(R);
        bool ok_mask = true;
        for (size_t r = 0; r < rows; r++) {
            double s = 0;
            for (size_t c = 0; c < rows; c++) {
                if (c > r) ok_mask = ok_mask && ch[r * rows + c] == 0.0f;
                s += ch[r * rows + c];
            }
            ok_mask = ok_mask && std::fabs(s - 1.0) <= 1e-5;
        }
        CHECK(ok_mask, "causal_mask + softmax_rows");
        group("rows", f);
    }

    // ----------------------------------------------- sums and transposes
    {
        int f = g_failures;
        const size_t rows = 300, cols = 33;
        auto x = iota(rows * cols, 1.0f, -40.0f);
        Matrix X = R.matrix_from_host(x, rows, cols);
        auto sr = R.matrix_sum_rows(X).to_host(R);
        auto sc = R.matrix_sum_cols(X).to_host(R);
        bool ok_r = true, ok_c = true;
        for (size_t r = 0; r < rows; r++) {
            double s = 0;
            for (size_t c = 0; c < cols; c++) s += x[r * cols + c];
            ok_r = ok_r && sr[r] == (float)s;
        }
        for (size_t c = 0; c < cols; c++) {
            double s = 0;
            for (size_t r = 0; r < rows; r++) s += x[r * cols + c];
            ok_c = ok_c && sc[c] == (float)s;
        }
        CHECK(ok_r, "matrix_sum_rows (integer data, exact)");
        CHECK(ok_c, "matrix_sum_cols (integer data, exact)");
        auto t = R.matrix_transpose(X);
        auto th = t.to_host(R);
        bool ok_t = t.rows() == cols && t.cols() == rows;
        for (size_t r = 0; r < rows && ok_t; r++)
            for (size_t c = 0; c < cols; c++) ok_t = ok_t && th[c * rows + r] == x[r * cols + c];
        CHECK(ok_t, "matrix_transpose");
        group("sums_transpose", f);
    }

    // ---------------------------------------------------- vector operations
    {
        int f = g_failures;
        const size_t n = 5000;
        auto a = iota(n, 1.0f, -48.0f), b = iota(n, 0.5f, 1.0f);
        Vector A = R.vector_from_host(a), B = R.vector_from_host(b);
        double s = 0, m = -1e300, d = 0;
        for (size_t i = 0; i < n; i++) {
            s += a[i];
            m = std::fmax(m, a[i]);
            d += (double)a[i] * b[i];
        }
        CHECK(A.sum(R) == (float)s, "Vector::sum (integer data, exact)");
        CHECK(A.max(R) == (float)m, "Vector::max");
        CHECK(std::fabs(A.dot(B, R) - d) <= 1e-6 * std::fabs(d) + 1e-3, "Vector::dot");
        Vector C = R.clone_vector(A);
        CHECK(A.equals(C, R), "Vector::equals (same)");
        C.add_scalar(1.0f, R);
        CHECK(!A.equals(C, R), "Vector::equals (different)");
        auto sum_v = R.vector_add(A, B).to_host(R);
        bool ok = true;
        for (size_t i = 0; i < n; i++) ok = ok && sum_v[i] == a[i] + b[i];
        CHECK(ok, "vector_add");
        auto sm_in = uniform(200, 9);
        Vector V = R.vector_from_host(sm_in);
        V.softmax(R);
        auto vh = V.to_host(R);
        double mx = -1e300, z = 0, e = 0;
        for (float v : sm_in) mx = std::fmax(mx, v);
        for (float v : sm_in) z += std::exp(v - mx);
        for (size_t i = 0; i < 200; i++) e = std::fmax(e, std::fabs(vh[i] - std::exp(sm_in[i] - mx) / z));
        CHECK(e <= 1e-5, "Vector::softmax");
        group("vectors", f);
    }

    // ------------------------------------------------------- conversions
    {
        int f = g_failures;
        std::vector<Vector> vs;
        for (int i = 0; i < 3; i++) vs.push_back(R.vector_from_host(iota(8, 1.0f, (float)(10 * i))));
        Matrix Z = R.vector_zip(vs);
        auto zh = Z.to_host(R);
        bool ok = Z.rows() == 3 && Z.cols() == 8;
        for (int i = 0; i < 3 && ok; i++) {
            auto want = iota(8, 1.0f, (float)(10 * i));
            for (int j = 0; j < 8; j++) ok = ok && zh[i * 8 + j] == want[j];
        }
        CHECK(ok, "vector_zip");
        auto parts = R.matrix_split(Z);
        ok = parts.size() == 3;
        for (size_t i = 0; i < parts.size() && ok; i++) ok = parts[i].to_host(R) == iota(8, 1.0f, (float)(10 * i));
        CHECK(ok, "matrix_split");
        Matrix Bc = R.broadcast(vs[1], 4);
        auto bh = Bc.to_host(R);
        ok = Bc.rows() == 4 && Bc.cols() == 8;
        for (int r = 0; r < 4 && ok; r++)
            for (int j = 0; j < 8; j++) ok = ok && bh[r * 8 + j] == iota(8, 1.0f, 10.0f)[j];
        CHECK(ok, "broadcast");
        Vector first = R.extract_vector(R.clone_matrix(Z));
        CHECK(first.to_host(R) == iota(8, 1.0f, 0.0f), "extract_vector (first row)");
        // matrix_slice: [4, 6] into 2x3 tiles, row-major over tiles.
        auto src = iota(24, 1.0f, 0.0f);
        for (int i = 0; i < 24; i++) src[i] = (float)i;
        Matrix S = R.matrix_from_host(src, 4, 6);
        auto tiles = R.matrix_slice(S, 3, 2);
        ok = tiles.size() == 4;
        for (size_t t = 0; t < tiles.size() && ok; t++) {
            auto th = tiles[t].to_host(R);
            const size_t tr = t / 2, tc = t % 2;
            for (size_t r = 0; r < 2; r++)
                for (size_t c = 0; c < 3; c++)
                    ok = ok && th[r * 3 + c] == src[(tr * 2 + r) * 6 + tc * 3 + c];
        }
        CHECK(ok, "matrix_slice");
        Vector flat = R.matrix_into_vector(R.clone_matrix(S));
        CHECK(flat.len() == 24 && flat.to_host(R) == src, "matrix_into_vector");
        Matrix col = R.vector_into_matrix(std::move(flat));
        CHECK(col.rows() == 24 && col.cols() == 1 && col.to_host(R) == src, "vector_into_matrix");
        group("conversions", f);
    }

    // ------------------------------------------------------- buffer pool
    {
        int f = g_failures;
        const size_t n = 12345;
        R.reserve_buffers(n, 2);
        DeviceBuffer a = R.get_uninit_buffer(n);
        float* p = a.ptr();
        R.recycle_buffer(std::move(a));
        DeviceBuffer b = R.get_uninit_buffer(n);
        CHECK(b.ptr() == p, "recycled buffer is reused");
        DeviceBuffer z = R.get_zerod_buffer(n);
        Vector zv(std::move(z));
        bool ok = true;
        for (float v : zv.to_host(R)) ok = ok && v == 0.0f;
        CHECK(ok, "get_zerod_buffer");
        Vector u = R.vector_from_host(iota(5, 1.0f, 1.0f)), w = R.vector_from_host(iota(3, 1.0f, 100.0f));
        DeviceBuffer cat = R.concat_buffers({&u.buffer(), &w.buffer()});
        Vector cv(std::move(cat));
        auto ch = cv.to_host(R);
        auto want = iota(5, 1.0f, 1.0f);
        auto w2 = iota(3, 1.0f, 100.0f);
        want.insert(want.end(), w2.begin(), w2.end());
        CHECK(ch == want, "concat_buffers");
        group("pool", f);
    }

    // ------------------------------------------------------ Linear and MLP
    {
        int f = g_failures;
        const size_t B = 17, I = 24, O = 12;
        auto x = uniform(B * I, 10), wv = uniform(I * O, 11), bv = uniform(O, 12);
        Linear lin(R.matrix_from_host(wv, I, O), R.vector_from_host(bv), Activation::Relu);
        Matrix X = R.matrix_from_host(x, B, I);
        auto y = lin.forward(X, nullptr, R, nullptr).to_host(R);
        std::vector<double> ref(B * O), err(B * O);
        for (size_t i = 0; i < B; i++)
            for (size_t j = 0; j < O; j++) {
                double z = bv[j];
                for (size_t k = 0; k < I; k++) z += (double)x[i * I + k] * wv[k * O + j];
                ref[i * O + j] = z > 0 ? z : 0;
            }
        for (size_t i = 0; i < B * O; i++) err[i] = y[i] - ref[i];
        CHECK(max_abs(err) <= 1e-4 * max_abs(ref), "Linear::forward (ReLU, bias)");
        std::vector<Linear> layers;
        layers.emplace_back(R.matrix_from_host(wv, I, O), std::nullopt, Activation::Identity);
        InferenceMLP mlp(std::move(layers), std::nullopt);
        auto y2 = mlp.forward(X, R).to_host(R);
        for (size_t i = 0; i < B; i++)
            for (size_t j = 0; j < O; j++) {
                double z = 0;
                for (size_t k = 0; k < I; k++) z += (double)x[i * I + k] * wv[k * O + j];
                err[i * O + j] = y2[i * O + j] - z;
            }
        CHECK(max_abs(err) <= 1e-4 * 10.0, "InferenceMLP::forward");
        group("executors", f);
    }

    // ---------------------------------------------------- runtime wrappers
    // The element-wise Matrix / Vector operations (matrix.rs:178-253,
    // vector_runtime.rs:76-117), the device-slice constructors, and the *_on
    // variants on a forked stream, against host f32 arithmetic (one rounding
    // per element: bit for bit), exact integer sums and an f64 product.
    {
        int f = g_failures;
        const size_t r = 7, c = 9, n = 5;
        const std::vector<float> ha = uniform(r * c, 81);
        std::vector<float> hb = uniform(r * c, 82);
        for (auto& v : hb) v = v < 0.0f ? v - 0.5f : v + 0.5f;  // away from zero
        auto host = [&](BinaryOp op) {
            std::vector<float> o(r * c);
            for (size_t i = 0; i < o.size(); i++) {
                const float x = ha[i], y = hb[i];
                o[i] = op == BinaryOp::Add ? x + y
                       : op == BinaryOp::Sub ? x - y
                       : op == BinaryOp::Mul ? x * y
                                             : x / y;
            }
            return o;
        };
        Matrix A = R.matrix_from_host(ha, r, c), B = R.matrix_from_host(hb, r, c);
        CHECK(R.matrix_add(A, B).to_host(R) == host(BinaryOp::Add), "matrix_add");
        CHECK(R.matrix_sub(A, B).to_host(R) == host(BinaryOp::Sub), "matrix_sub");
        CHECK(R.matrix_mul(A, B).to_host(R) == host(BinaryOp::Mul), "matrix_mul");
        CHECK(R.matrix_div(A, B).to_host(R) == host(BinaryOp::Div), "matrix_div");
        Vector va = R.vector_from_host(ha), vb = R.vector_from_host(hb);
        CHECK(R.vector_add(va, vb).to_host(R) == host(BinaryOp::Add), "vector_add");
        CHECK(R.vector_sub(va, vb).to_host(R) == host(BinaryOp::Sub), "vector_sub");
        CHECK(R.vector_mul(va, vb).to_host(R) == host(BinaryOp::Mul), "vector_mul");
        CHECK(R.vector_div(va, vb).to_host(R) == host(BinaryOp::Div), "vector_div");
        CHECK(R.vector_binary(va, vb, BinaryOp::Div).to_host(R) == host(BinaryOp::Div),
              "vector_binary");
        CHECK(R.matrix_from_device(A.slice(), r, c).to_host(R) == ha, "matrix_from_device");
        CHECK(R.vector_from_device(vb.slice()).to_host(R) == hb, "vector_from_device");

        // *_on on a forked stream, joined before the results are read.
        std::vector<float> hi(r * c), hw = uniform(c * n, 83), hrow = uniform(c, 84);
        for (size_t i = 0; i < hi.size(); i++) hi[i] = (float)((int)(i * 7 % 23) - 11);
        Matrix I = R.matrix_from_host(hi, r, c), W = R.matrix_from_host(hw, c, n);
        Matrix out = R.new_uninit_matrix(r, n), M2 = R.clone_matrix(A), M3 = R.clone_matrix(A);
        Vector row = R.vector_from_host(hrow), v2 = R.clone_vector(va);
        auto st = R.create_extra_streams(1);
        R.fork_streams(st);
        const CudaStream* s = &st[0];
        Matrix cm = R.clone_matrix_on(A, s);
        Vector cv = R.clone_vector_on(vb, s);
        Vector sums = R.matrix_sum_rows_on(I, s);
        Matrix prod = R.matrix_binary_on(s, A, B, BinaryOp::Mul);
        R.matrix_multiply_into_on(s, A, W, out);
        v2.scale_on(2.0f, R, s);
        M2.binary_assign_on(B, BinaryOp::Sub, R, s);
        M3.binary_assign_by_rows_on(row, BinaryOp::Add, R, s);
        R.join_streams(st);
        R.sync();
        CHECK(cm.to_host(R) == ha && cv.to_host(R) == hb, "clone_*_on");
        std::vector<float> want_sums(r, 0.0f);
        for (size_t i = 0; i < r; i++)
            for (size_t j = 0; j < c; j++) want_sums[i] += hi[i * c + j];
        CHECK(sums.to_host(R) == want_sums, "matrix_sum_rows_on (integers, exact)");
        CHECK(prod.to_host(R) == host(BinaryOp::Mul), "matrix_binary_on");
        CHECK(M2.to_host(R) == host(BinaryOp::Sub), "binary_assign_on");
        std::vector<float> want_row(r * c), want_scale(r * c);
        for (size_t i = 0; i < r * c; i++) {
            want_row[i] = ha[i] + hrow[i % c];
            want_scale[i] = ha[i] * 2.0f;
        }
        CHECK(M3.to_host(R) == want_row, "binary_assign_by_rows_on");
        CHECK(v2.to_host(R) == want_scale, "scale_on");
        const auto got = out.to_host(R);
        double err = 0.0, big = 0.0;
        for (size_t i = 0; i < r; i++)
            for (size_t j = 0; j < n; j++) {
                double s64 = 0.0;
                for (size_t k = 0; k < c; k++) s64 += (double)ha[i * c + k] * hw[k * n + j];
                err = std::max(err, std::fabs(got[i * n + j] - s64));
                big = std::max(big, std::fabs(s64));
            }
        CHECK(err / big <= 1e-5, "matrix_multiply_into_on");
        group("runtime wrappers", f);
    }

    // ----------------------------------------------------- cross attention
    // Attention::forward / forward_mask with query and key/value inputs of
    // different row counts (attention.rs:221-241): norm(Xq + softmax(Q K^T /
    // sqrt(d)) V), Q from Xq, K and V from Xkv, against a double-precision
    // host evaluation; with the Q/K/V projections batched and on three
    // forked streams (bit-identical to each other).
    {
        int f = g_failures;
        const size_t Sq = 40, Sk = 72, H = 32, D = 16;
        auto host_lin = [&](size_t in, size_t out, uint64_t seed, std::vector<float>& w,
                            std::vector<float>& b) {
            w = uniform(in * out, seed);
            for (auto& v : w) v *= 0.3f;
            b = uniform(out, seed + 100);
        };
        std::vector<float> wq, bq, wk, bk, wv, bv;
        host_lin(H, D, 71, wq, bq);
        host_lin(H, D, 72, wk, bk);
        host_lin(H, H, 73, wv, bv);
        const std::vector<float> xq = uniform(Sq * H, 74), xkv = uniform(Sk * H, 75);
        auto make = [&](bool streams) {
            auto lin = [&](const std::vector<float>& w, const std::vector<float>& b, size_t in,
                           size_t out) {
                return Linear(R.matrix_from_host(w, in, out), R.vector_from_host(b),
                              Activation::Identity);
            };
            Normalization n;
            n.kind = NormType::Layer;
            std::optional<std::vector<CudaStream>> s;
            if (streams) s = R.create_extra_streams(3);
            return Attention(lin(wq, bq, H, D), lin(wk, bk, H, D), lin(wv, bv, H, H), std::move(s),
                             std::move(n));
        };
        // host reference
        auto proj = [](const std::vector<float>& x, size_t rows, size_t in,
                       const std::vector<float>& w, const std::vector<float>& b, size_t out) {
            std::vector<double> y(rows * out);
            for (size_t r = 0; r < rows; r++)
                for (size_t c = 0; c < out; c++) {
                    double s = b[c];
                    for (size_t k = 0; k < in; k++) s += (double)x[r * in + k] * w[k * out + c];
                    y[r * out + c] = s;
                }
            return y;
        };
        const auto Q = proj(xq, Sq, H, wq, bq, D), K = proj(xkv, Sk, H, wk, bk, D),
                   V = proj(xkv, Sk, H, wv, bv, H);
        auto reference = [&](bool mask) {
            std::vector<double> out(Sq * H);
            const double scale = 1.0 / std::sqrt((double)D);
            for (size_t r = 0; r < Sq; r++) {
                std::vector<double> p(Sk);
                double m = -1e300;
                for (size_t c = 0; c < Sk; c++) {
                    double s = 0.0;
                    for (size_t k = 0; k < D; k++) s += Q[r * D + k] * K[c * D + k];
                    p[c] = (mask && c > r) ? -1e300 : s * scale;
                    m = std::max(m, p[c]);
                }
                double z = 0.0;
                for (size_t c = 0; c < Sk; c++) z += (p[c] = (p[c] <= -1e299) ? 0.0 : std::exp(p[c] - m));
                std::vector<double> a(H);
                for (size_t h = 0; h < H; h++) {
                    double s = 0.0;
                    for (size_t c = 0; c < Sk; c++) s += p[c] / z * V[c * H + h];
                    a[h] = xq[r * H + h] + s;
                }
                double mu = 0.0, var = 0.0;
                for (double t : a) mu += t;
                mu /= H;
                for (double t : a) var += (t - mu) * (t - mu);
                var /= H;
                for (size_t h = 0; h < H; h++) out[r * H + h] = (a[h] - mu) / std::sqrt(var + 1e-5);
            }
            return out;
        };
        Matrix Xq = R.matrix_from_host(xq, Sq, H), Xkv = R.matrix_from_host(xkv, Sk, H);
        for (bool mask : {false, true}) {
            const auto want = reference(mask);
            std::vector<float> got[2];
            for (int streams = 0; streams < 2; streams++) {
                Attention attn = make(streams == 1);
                Matrix y = mask ? attn.forward_mask(Xq, Xkv, R) : attn.forward(Xq, Xkv, R);
                CHECK(y.rows() == Sq && y.cols() == H, "cross attention shape");
                got[streams] = y.to_host(R);
            }
            double err = 0.0, big = 0.0;
            for (size_t i = 0; i < want.size(); i++) {
                err = std::max(err, std::fabs(got[0][i] - want[i]));
                big = std::max(big, std::fabs(want[i]));
            }
            CHECK(err / big <= 1e-4, mask ? "cross attention (masked) vs host" :
                                            "cross attention vs host");
            CHECK(got[0] == got[1], "cross attention: forked streams = batched");
        }
        group("cross attention", f);
    }

    // ---------------------------------------------------------- checkpoint
    // Shapes only the C++ API can hold: a three-layer feed-forward network
    // with a residual, query/key narrower than the embedding.
    {
        int f = g_failures;
        const char* tmp = std::getenv("TMPDIR");
        const std::string base = std::string(tmp && *tmp ? tmp : "/tmp") + "/oxforge_ckpt_" +
                                 std::to_string((long)getpid());
        const size_t S = 24, H = 32, QK = 16, F = 48, O = 8;
        auto lin = [&](size_t in, size_t out, uint64_t seed, bool bias, Activation a) {
            auto w = uniform(in * out, seed);
            for (auto& v : w) v *= 0.3f;
            std::optional<Vector> b;
            if (bias) b = R.vector_from_host(uniform(out, seed + 100));
            return Linear(R.matrix_from_host(w, in, out), std::move(b), a);
        };
        auto layers = [&]() {
            std::vector<Linear> l;
            l.push_back(lin(H, F, 31, true, Activation::Gelu));
            l.push_back(lin(F, F, 32, false, Activation::Silu));
            l.push_back(lin(F, H, 33, true, Activation::Identity));
            return l;
        };
        auto norm = [&](uint64_t seed) {
            Normalization n;
            n.kind = NormType::Layer;
            auto g = uniform(H, seed);
            for (auto& v : g) v = 1.0f + 0.1f * v;
            n.gamma = R.vector_from_host(g);
            n.beta = R.vector_from_host(uniform(H, seed + 1));
            return n;
        };
        encoder::InferenceTransformer t(
            lin(H, QK, 21, true, Activation::Identity), lin(H, QK, 22, true, Activation::Identity),
            lin(H, H, 23, false, Activation::Identity), R.matrix_from_host(uniform(S * H, 24), S, H),
            InferenceMLP(layers(), std::make_pair((size_t)0, (size_t)3)),
            lin(H, O, 25, true, Activation::Identity), std::nullopt, NormType::Layer, norm(40),
            norm(50));
        Matrix X = R.matrix_from_host(uniform(S * H, 26), S, H);
        auto want = t.forward(X, R).to_host(R);
        checkpoint::dump_transformer(t, base, R);
        const checkpoint::TransformerMetadata md = checkpoint::read_transformer_metadata(base);
        CHECK(md.feed_forward.layers.size() == 3 && md.feed_forward.residual &&
                  md.feed_forward.residual->end == 3 && md.query.output_neurons == QK &&
                  md.norm2_beta && md.feed_forward.layers[1].activation == Activation::Silu,
              "transformer metadata");
        uint64_t bytes = 0;
        CHECK(checkpoint::inspect(base + ".toml", &bytes) == "transformer" &&
                  bytes == md.norm2_beta->byte_end,
              "inspect");
        encoder::InferenceTransformer back = checkpoint::load_transformer(base, R);
        CHECK(back.forward(X, R).to_host(R) == want, "load_transformer forward bit-identical");
        encoder::TrainingTransformer train = checkpoint::load_training_transformer(base, R);
        CHECK(train.forward(X, R).to_host(R) == want, "load_training_transformer forward");
        bool refused = false;
        try {
            checkpoint::load_linear(base, R);
        } catch (const Error& e) {
            refused = e.status() == FORGE_EINVAL;
        }
        CHECK(refused, "model type mismatch refused");
        Linear l = lin(H, O, 60, true, Activation::Relu);
        checkpoint::dump_linear(l, base + "_lin.toml", R);
        Linear l2 = checkpoint::load_linear(base + "_lin", R);
        CHECK(l2.weights().to_host(R) == l.weights().to_host(R) &&
                  l2.bias()->to_host(R) == l.bias()->to_host(R) &&
                  l2.activation() == Activation::Relu,
              "Linear round trip");
        for (const char* suffix : {".toml", ".bin", "_lin.toml", "_lin.bin"})
            std::remove((base + suffix).c_str());
        group("checkpoint", f);
    }

    // ----------------------------------------------- spans and row views
    {
        int f = g_failures;
        const size_t rows = 6, cols = 1000;
        std::vector<float> h = uniform(rows * cols, 11);
        for (float& x : h) x *= 4.0f;
        Matrix m = R.matrix_from_host(h, rows, cols);
        std::vector<VectorView> views = m.row_views();
        CHECK(views.size() == rows, "row_views count");
        for (auto& v : views) CHECK(v.len() == cols, "row view length");
        // map_sum of every row with six functors (checked against the oracle
        // by the Python test), plus exact cases checked here.
        const MapFn fns[] = {MapFn::identity(), MapFn::scale(0.5f), MapFn::add(1.25f),
                             MapFn::half_square(), MapFn::exp_shift(0.3f),
                             MapFn::of(FORGE_MAP_GELU)};
        std::vector<float> sums;
        for (auto& v : views)
            for (const MapFn& fn : fns) sums.push_back(v.map_sum(R, fn));
        for (size_t r = 0; r < rows; r++) {
            double ref = 0;
            for (size_t c = 0; c < cols; c++) ref += h[r * cols + c];
            CHECK(std::fabs(sums[r * 6] - views[r].sum(R)) <= 1e-6 * (1 + std::fabs(ref)),
                  "map_sum(identity) == sum");
        }
        for (auto& v : views) v.softmax(R);
        std::vector<float> sm = m.to_host(R);
        for (size_t r = 0; r < rows; r++) {
            double mx = -1e30, z = 0, t = 0, err = 0;
            for (size_t c = 0; c < cols; c++) mx = std::fmax(mx, h[r * cols + c]);
            for (size_t c = 0; c < cols; c++) z += std::exp((double)h[r * cols + c] - mx);
            for (size_t c = 0; c < cols; c++) {
                double ref = std::exp((double)h[r * cols + c] - mx) / z;
                err = std::fmax(err, std::fabs(ref - sm[r * cols + c]));
                t += sm[r * cols + c];
            }
            CHECK(err <= 1e-5 && std::fabs(t - 1.0) <= 1e-4, "VectorView::softmax row");
        }
        if (!dump_dir.empty()) {
            dump(dump_dir + "/spans_input.f32", h);
            dump(dump_dir + "/spans_softmax.f32", sm);
            dump(dump_dir + "/spans_map_sum.f32", sums);
        }

        // Vector spans (vector.rs:11-17), copies, chunks and concatenation.
        std::vector<float> hv = iota(1000);
        Vector vec = R.vector_from_host(hv);
        DeviceSpan sp = vec.span(10, 100);
        CHECK(sp.len() == 100 && vec.as_span().len() == 1000, "span lengths");
        DeviceBuffer copy = sp.to_buffer(R);
        std::vector<float> got(100);
        check(forge_memcpy_d2h(R.raw(), got.data(), copy.slice(), 100), "span copy");
        CHECK(std::equal(got.begin(), got.end(), hv.begin() + 10), "DeviceSpan::to_buffer");
        float exact = 0, mx = -1e30f;
        for (size_t i = 10; i < 110; i++) exact += hv[i], mx = std::fmax(mx, hv[i]);
        CHECK(sp.sum(R) == exact && sp.max(R) == mx, "span sum/max (integers: exact)");
        CHECK(sp.map_sum(R, MapFn::scale(2.0f)) == 2 * exact, "span map_sum exact");
        std::vector<DeviceSpan> ch = DeviceSpan::chunks(vec.buffer(), 300);
        CHECK(ch.size() == 4 && ch[3].len() == 100 && ch[0].len() == 300, "chunks");
        DeviceBuffer cat = R.concat_buffers_from_span({ch[3], ch[0]});
        std::vector<float> hc(400);
        check(forge_memcpy_d2h(R.raw(), hc.data(), cat.slice(), 400), "concat copy");
        CHECK(std::equal(hc.begin(), hc.begin() + 100, hv.begin() + 900) &&
                  std::equal(hc.begin() + 100, hc.end(), hv.begin()),
              "concat_buffers_from_span");
        DeviceSpan empty = vec.span(1000, 0);
        CHECK(empty.sum(R) == 0.0f && empty.max(R) == -3.40282347e38f &&
                  empty.map_sum(R, MapFn::add(1.0f)) == 0.0f,
              "empty span identities");
        bool refused = false;
        try {
            (void)vec.span(990, 20);
        } catch (const Error& e) {
            refused = e.status() == FORGE_EINVAL;
        }
        CHECK(refused, "span past the buffer refused");
        // A mutable sub-span changes only its own range.
        DeviceSpanMut mut = DeviceSpanMut::from_buffer(vec.buffer(), 100, 50);
        mut.scale(3.0f, R);
        mut.for_each(R, MapFn::add(1.0f));
        std::vector<float> after = vec.to_host(R);
        bool ok = true;
        for (size_t i = 0; i < 1000; i++) {
            float want = (i >= 100 && i < 150) ? hv[i] * 3.0f + 1.0f : hv[i];
            ok = ok && after[i] == want;
        }
        CHECK(ok, "DeviceSpanMut::for_each on a sub-span");
        group("spans", f);
    }

    // ------------------------------------------- reference API members
    {
        int f = g_failures;
        // InitType::is_zero (runtime.rs:14-21).
        CHECK(InitType(InitType::Zero).is_zero() && !InitType(InitType::Sequence).is_zero() &&
                  !InitType(InitType::Reserve).is_zero() && !InitType(InitType::Random).is_zero(),
              "InitType::is_zero");
        // MetadataCursor (metadata.rs:20-68): consecutive f32 byte ranges.
        MetadataCursor c;
        MatrixMetadata m0 = c.matrix(3, 5);
        VectorMetadata v0 = c.vector(7);
        MatrixMetadata m1 = c.matrix(0, 9);
        CHECK(m0.byte_start == 0 && m0.byte_end == 60 && v0.byte_start == 60 &&
                  v0.byte_end == 88 && m1.byte_start == 88 && m1.byte_end == 88 &&
                  c.data_bytes() == 88,
              "MetadataCursor ranges");
        bool overflow = false;
        try {
            (void)c.matrix(SIZE_MAX / 2, 3);
        } catch (const Error& e) {
            overflow = e.status() == FORGE_EINVAL;
        }
        CHECK(overflow, "MetadataCursor element overflow refused");
        // get_u32_uninit_buffer (runtime.rs:57-60) and Vector::equals through
        // it (vector.rs:117-136), with the mismatch in the last element.
        DeviceBufferU32 u = R.get_u32_uninit_buffer(5);
        CHECK(u.len() == 5 && u.ptr() != nullptr, "get_u32_uninit_buffer");
        CHECK(R.get_u32_uninit_buffer(0).is_empty(), "empty u32 buffer");
        auto hv = uniform(3000, 21);
        Vector a = R.vector_from_host(hv);
        Vector b = R.vector_from_host(hv);
        CHECK(a.equals(b, R), "equals on equal vectors");
        hv[2999] += 1.0f;
        Vector c2 = R.vector_from_host(hv);
        CHECK(!a.equals(c2, R), "equals sees the last element");
        forge_slice_u32 count = u.slice();
        check(forge_compare_u32(R.raw(), nullptr, a.slice(), c2.slice(), 3000, count),
              "compare_u32");
        CHECK(u.to_host(R)[0] == 1u, "compare_u32 mismatch count");
        // span_to_buffer_async (runtime.rs:184-186).
        DeviceSpan sp = a.span(100, 250);
        DeviceBuffer copy = R.span_to_buffer_async(sp);
        std::vector<float> got(250);
        check(forge_memcpy_d2h(R.raw(), got.data(), copy.slice(), 250), "copy to host");
        auto want = b.to_host(R);
        CHECK(copy.len() == 250 && std::equal(got.begin(), got.end(), want.begin() + 100),
              "span_to_buffer_async");
        // with_loss constructors (mlp.rs:37-51, 180-184, 214-219).
        auto lin = [&](size_t in, size_t out, uint64_t seed) {
            return Linear(R.matrix_from_host(uniform(in * out, seed), in, out), std::nullopt,
                          Activation::Identity);
        };
        std::vector<Linear> l1, l2, l3;
        l1.push_back(lin(8, 16, 31));
        l2.push_back(lin(8, 16, 32));
        l3.push_back(lin(8, 16, 33));
        MlpExecutor e = MlpExecutor::with_loss(std::move(l1), std::nullopt, Loss::MeanSquaredError);
        InferenceMLP i = InferenceMLP::with_loss(std::move(l2), std::nullopt, Loss::MeanSquaredError);
        TrainingMlp t = TrainingMlp::with_loss(std::move(l3), std::nullopt, Loss::MeanSquaredError);
        CHECK(e.len() == 1 && e.loss() == Loss::MeanSquaredError &&
                  i.loss() == Loss::MeanSquaredError && t.loss() == Loss::MeanSquaredError,
              "with_loss constructors");
        bool bad_range = false;
        try {
            std::vector<Linear> l4;
            l4.push_back(lin(8, 8, 34));
            (void)MlpExecutor::with_loss(std::move(l4), std::make_pair<size_t, size_t>(1, 1),
                                         Loss::MeanSquaredError);
        } catch (const Error& err) {
            bad_range = err.status() == FORGE_EINVAL;
        }
        CHECK(bad_range, "with_loss refuses an empty residual range");
        group("reference API members", f);
    }

    R.sync();
    std::printf("%s: %d failed check(s)\n", g_failures ? "FAILED" : "OK", g_failures);
    return g_failures ? 1 : 0;
}
