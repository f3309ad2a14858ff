// net_capi.cpp -- C entry points of include/oxforge_net.h over the C++
// executors.  Exceptions become status codes; parameters are copied into
// model-owned device buffers at creation.
#include <cstring>
#include <new>

#include "oxforge_net.h"
#include "oxforge_checkpoint.hpp"
#include "oxforge_net.hpp"

extern "C" void forge_internal_set_error(const char* message);

using namespace oxforge;

struct forge_net_model {
    // Declared first so it is destroyed last: every Matrix below returns its
    // buffer to the pool through this wrapper.
    std::unique_ptr<CudaRuntime> rt;
    std::unique_ptr<Linear> linear;
    std::unique_ptr<InferenceMLP> imlp;
    std::unique_ptr<TrainingMlp> tmlp;
    std::unique_ptr<encoder::InferenceTransformer> enc_inf;
    std::unique_ptr<encoder::TrainingTransformer> enc_train;
    std::unique_ptr<decoder::InferenceTransformer> dec_inf;
    forge_transformer_desc desc{};
};

namespace {

template <typename F>
forge_status guard(F&& f) {
    try {
        f();
        return FORGE_OK;
    } catch (const Error& e) {
        forge_internal_set_error(e.what());
        return e.status();
    } catch (const std::bad_alloc&) {
        forge_internal_set_error("host allocation failed");
        return FORGE_ENOMEM;
    } catch (const std::exception& e) {
        forge_internal_set_error(e.what());
        return FORGE_EINVAL;
    }
}

void require(bool cond, const char* what) {
    if (!cond) throw Error(FORGE_EINVAL, what);
}

void need(forge_slice s, size_t n, const char* what) {
    if (n > 0 && (!s.ptr || s.len < n))
        throw Error(FORGE_EINVAL, std::string(what) + ": slice too short");
}

bool present(forge_slice s) { return s.ptr != nullptr; }

// Copies caller device data into a model-owned Matrix / Vector.
Matrix own_matrix(CudaRuntime& rt, forge_slice s, size_t rows, size_t cols, const char* what) {
    need(s, rows * cols, what);
    return rt.matrix_from_device(s, rows, cols);
}

std::optional<Vector> own_vector(CudaRuntime& rt, forge_slice s, size_t n, const char* what) {
    if (!present(s)) return std::nullopt;
    need(s, n, what);
    return rt.vector_from_device(forge_slice{s.ptr, n});
}

Activation activation_of(int a) {
    require(a >= 0 && a <= 3, "unknown activation");
    return (Activation)a;
}

void copy_out(CudaRuntime& rt, forge_slice dst, const Matrix& src, const char* what) {
    need(dst, src.len(), what);
    check(forge_memcpy_d2d(rt.raw(), nullptr, dst, src.slice(), src.len()), what);
}

void copy_out(CudaRuntime& rt, forge_slice dst, const Vector& src, const char* what) {
    need(dst, src.len(), what);
    check(forge_memcpy_d2d(rt.raw(), nullptr, dst, src.slice(), src.len()), what);
}

forge_net_model* new_model(forge_runtime* rt) {
    auto* m = new forge_net_model();
    m->rt = CudaRuntime::borrow(rt);
    return m;
}

}  // namespace

extern "C" forge_status forge_net_model_destroy(forge_net_model* m) {
    if (!m) return FORGE_OK;
    return guard([&] {
        if (m->rt) m->rt->sync();
        delete m;
    });
}

// ================================================================== Linear

extern "C" forge_status forge_net_linear_create(forge_runtime* rt, forge_slice weights, size_t in,
                                                size_t out, forge_slice bias, int activation,
                                                forge_net_model** out_model) {
    if (!rt || !out_model) return FORGE_EINVAL;
    *out_model = nullptr;
    return guard([&] {
        std::unique_ptr<forge_net_model> m(new_model(rt));
        Matrix w = own_matrix(*m->rt, weights, in, out, "linear weights");
        std::optional<Vector> b = own_vector(*m->rt, bias, out, "linear bias");
        m->linear.reset(new Linear(std::move(w), std::move(b), activation_of(activation)));
        *out_model = m.release();
    });
}

extern "C" forge_status forge_net_linear_forward(forge_net_model* m, forge_slice x, size_t rows,
                                                 forge_slice residual, forge_slice y,
                                                 forge_slice pre_out) {
    if (!m || !m->linear) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        Linear& lin = *m->linear;
        const size_t in = lin.weights().rows(), out = lin.weights().cols();
        Matrix X = own_matrix(rt, x, rows, in, "linear input");
        std::optional<Matrix> R;
        if (present(residual)) R = own_matrix(rt, residual, rows, out, "linear residual");
        std::optional<Matrix> pre;
        if (present(pre_out)) pre = rt.new_uninit_matrix(rows, out);
        Matrix Y = lin.forward_keep(X, R ? &*R : nullptr, pre ? &*pre : nullptr, rt, nullptr);
        copy_out(rt, y, Y, "linear output");
        if (pre) copy_out(rt, pre_out, *pre, "linear pre-activation");
        rt.sync();
    });
}

extern "C" forge_status forge_net_linear_backward(forge_net_model* m, forge_slice pre,
                                                  forge_slice dy, size_t rows, forge_slice g_out,
                                                  forge_slice db_out) {
    if (!m || !m->linear) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        Linear& lin = *m->linear;
        const size_t out = lin.weights().cols();
        Matrix DY = own_matrix(rt, dy, rows, out, "linear dy");
        std::optional<Matrix> P;
        if (present(pre)) P = own_matrix(rt, pre, rows, out, "linear pre-activation");
        auto gb = lin.backward(P ? &*P : nullptr, DY, rt, nullptr);
        copy_out(rt, g_out, gb.first, "linear gradient");
        if (present(db_out) && gb.second) copy_out(rt, db_out, *gb.second, "linear bias gradient");
        rt.sync();
    });
}

extern "C" forge_status forge_net_linear_input_gradient(forge_net_model* m, forge_slice g,
                                                        size_t rows, forge_slice dx) {
    if (!m || !m->linear) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        Linear& lin = *m->linear;
        Matrix G = own_matrix(rt, g, rows, lin.weights().cols(), "linear gradient");
        Matrix DX = lin.input_gradient(G, rt, nullptr);
        copy_out(rt, dx, DX, "linear input gradient");
        rt.sync();
    });
}

extern "C" forge_status forge_net_linear_learn(forge_net_model* m, forge_slice x, forge_slice g,
                                               forge_slice db, size_t rows, float lr) {
    if (!m || !m->linear) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        Linear& lin = *m->linear;
        Matrix X = own_matrix(rt, x, rows, lin.weights().rows(), "linear input");
        Matrix G = own_matrix(rt, g, rows, lin.weights().cols(), "linear gradient");
        std::optional<Vector> DB = own_vector(rt, db, lin.weights().cols(), "linear bias gradient");
        lin.learn(X, G, DB ? &*DB : nullptr, lr, rt, nullptr);
        rt.sync();
    });
}

extern "C" forge_status forge_net_linear_loss_rows(forge_runtime* rt_raw, forge_slice output,
                                                   forge_slice target, size_t rows, size_t cols,
                                                   forge_slice loss) {
    if (!rt_raw) return FORGE_EINVAL;
    return guard([&] {
        auto rt = CudaRuntime::borrow(rt_raw);
        {
            Matrix O = own_matrix(*rt, output, rows, cols, "loss output");
            Matrix T = own_matrix(*rt, target, rows, cols, "loss target");
            Vector L = Linear::loss_rows(O, T, *rt, nullptr);
            copy_out(*rt, loss, L, "loss rows");
            rt->sync();
        }
    });
}

extern "C" forge_status forge_net_linear_param(forge_net_model* m, int which, forge_slice* out) {
    if (!m || !m->linear || !out) return FORGE_EINVAL;
    return guard([&] {
        if (which == 0) *out = m->linear->weights().slice();
        else if (which == 1) *out = m->linear->bias() ? m->linear->bias()->slice() : forge_slice{nullptr, 0};
        else throw Error(FORGE_EINVAL, "which must be 0 (weights) or 1 (bias)");
    });
}

// ===================================================================== MLP

extern "C" forge_status forge_net_mlp_create(forge_runtime* rt, size_t n_layers, const size_t* dims,
                                             const int* activations, const forge_slice* weights,
                                             const forge_slice* biases, long res_start,
                                             long res_end, int training,
                                             forge_net_model** out_model) {
    if (!rt || !out_model || !dims || !activations || !weights || n_layers == 0)
        return FORGE_EINVAL;
    *out_model = nullptr;
    return guard([&] {
        std::unique_ptr<forge_net_model> m(new_model(rt));
        std::vector<Linear> layers;
        for (size_t i = 0; i < n_layers; i++) {
            Matrix w = own_matrix(*m->rt, weights[i], dims[i], dims[i + 1], "mlp weights");
            std::optional<Vector> b =
                biases ? own_vector(*m->rt, biases[i], dims[i + 1], "mlp bias") : std::nullopt;
            layers.emplace_back(std::move(w), std::move(b), activation_of(activations[i]));
        }
        std::optional<std::pair<size_t, size_t>> res;
        if (res_start >= 0) res = std::make_pair((size_t)res_start, (size_t)res_end);
        if (training) m->tmlp.reset(new TrainingMlp(std::move(layers), res));
        else m->imlp.reset(new InferenceMLP(std::move(layers), res));
        *out_model = m.release();
    });
}

static MlpExecutor& mlp_exec(forge_net_model* m) {
    if (m->tmlp) return m->tmlp->executor();
    if (m->imlp) return m->imlp->executor();
    throw Error(FORGE_EINVAL, "model is not an MLP");
}

extern "C" forge_status forge_net_mlp_forward(forge_net_model* m, forge_slice x, size_t rows,
                                              forge_slice y) {
    if (!m) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        MlpExecutor& ex = mlp_exec(m);
        Matrix X = own_matrix(rt, x, rows, ex.layers().front().weights().rows(), "mlp input");
        Matrix Y = m->tmlp ? m->tmlp->forward(std::move(X), rt) : m->imlp->forward(X, rt);
        copy_out(rt, y, Y, "mlp output");
        rt.sync();
    });
}

extern "C" forge_status forge_net_mlp_backward(forge_net_model* m, forge_slice dy, size_t rows,
                                               float lr, forge_slice dx) {
    if (!m || !m->tmlp) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        MlpExecutor& ex = mlp_exec(m);
        Matrix DY = own_matrix(rt, dy, rows, ex.layers().back().weights().cols(), "mlp dy");
        Matrix DX = m->tmlp->backward(DY, lr, rt);
        if (present(dx)) copy_out(rt, dx, DX, "mlp input gradient");
        rt.sync();
    });
}

extern "C" forge_status forge_net_mlp_param(forge_net_model* m, size_t layer, int which,
                                            forge_slice* out) {
    if (!m || !out) return FORGE_EINVAL;
    return guard([&] {
        MlpExecutor& ex = mlp_exec(m);
        require(layer < ex.len(), "layer index out of range");
        Linear& lin = ex.layers()[layer];
        if (which == 0) *out = lin.weights().slice();
        else *out = lin.bias() ? lin.bias()->slice() : forge_slice{nullptr, 0};
    });
}

// ============================================================= transformer

namespace {

Normalization make_norm(CudaRuntime& rt, NormType kind, forge_slice gamma, forge_slice beta,
                        size_t hidden) {
    Normalization n;
    n.kind = kind;
    n.gamma = own_vector(rt, gamma, hidden, "norm gamma");
    if (kind == NormType::Layer) n.beta = own_vector(rt, beta, hidden, "norm beta");
    return n;
}

struct Parts {
    Attention* attention = nullptr;
    Normalization* norm2 = nullptr;
    Matrix* position = nullptr;
    MlpExecutor* ffn = nullptr;
    Linear* output = nullptr;
};

Parts parts_of(forge_net_model* m) {
    Parts p;
    if (m->enc_train) {
        p.attention = &m->enc_train->attention();
        p.norm2 = &m->enc_train->norm2();
        p.position = &m->enc_train->position();
        p.ffn = &m->enc_train->fcs().executor();
        p.output = &m->enc_train->output();
    } else {
        InferenceBlock& b = m->enc_inf ? m->enc_inf->block() : m->dec_inf->block();
        p.attention = &b.attention();
        p.norm2 = &b.norm2();
        p.position = &b.position();
        p.ffn = &b.fcs().executor();
        p.output = &b.output();
    }
    return p;
}

forge_slice opt(const std::optional<Vector>& v) { return v ? v->slice() : forge_slice{nullptr, 0}; }

}  // namespace

extern "C" forge_status forge_net_transformer_create(forge_runtime* rt,
                                                     const forge_transformer_desc* d,
                                                     const forge_slice* params,
                                                     forge_net_model** out_model) {
    if (!rt || !d || !params || !out_model) return FORGE_EINVAL;
    *out_model = nullptr;
    return guard([&] {
        std::unique_ptr<forge_net_model> m(new_model(rt));
        CudaRuntime& r = *m->rt;
        m->desc = *d;
        const size_t S = d->seq, H = d->hidden, F = d->ffn, O = d->out;
        require(S && H && F && O, "transformer dims must be non-zero");
        require(d->norm_type == 0 || d->norm_type == 1, "norm_type must be 0 (Rms) or 1 (Layer)");
        const NormType nt = d->norm_type == 0 ? NormType::Rms : NormType::Layer;
        auto lin = [&](int w, int b, size_t in, size_t out, Activation a) {
            return Linear(own_matrix(r, params[w], in, out, "transformer weights"),
                          own_vector(r, params[b], out, "transformer bias"), a);
        };
        Linear q = lin(FORGE_TP_WQ, FORGE_TP_BQ, H, H, Activation::Identity);
        Linear k = lin(FORGE_TP_WK, FORGE_TP_BK, H, H, Activation::Identity);
        Linear v = lin(FORGE_TP_WV, FORGE_TP_BV, H, H, Activation::Identity);
        Matrix pos = own_matrix(r, params[FORGE_TP_POS], S, H, "position matrix");
        std::vector<Linear> ffn;
        ffn.push_back(lin(FORGE_TP_W1, FORGE_TP_B1, H, F, activation_of(d->ffn_activation)));
        ffn.push_back(lin(FORGE_TP_W2, FORGE_TP_B2, F, H, Activation::Identity));
        Linear o = lin(FORGE_TP_WO, FORGE_TP_BO, H, O, Activation::Identity);
        Normalization n1 = make_norm(r, nt, params[FORGE_TP_G1], params[FORGE_TP_BE1], H);
        Normalization n2 = make_norm(r, nt, params[FORGE_TP_G2], params[FORGE_TP_BE2], H);
        std::optional<std::vector<CudaStream>> streams;
        if (d->qkv_streams) streams = r.create_extra_streams(3);
        switch (d->kind) {
        case FORGE_TK_ENCODER_INFERENCE:
            m->enc_inf.reset(new encoder::InferenceTransformer(
                std::move(q), std::move(k), std::move(v), std::move(pos),
                InferenceMLP(std::move(ffn), std::nullopt), std::move(o), std::move(streams), nt,
                std::move(n1), std::move(n2)));
            break;
        case FORGE_TK_ENCODER_TRAINING:
            m->enc_train.reset(new encoder::TrainingTransformer(
                std::move(q), std::move(k), std::move(v), std::move(pos),
                TrainingMlp(std::move(ffn), std::nullopt), std::move(o), nt, std::move(n1),
                std::move(n2)));
            break;
        case FORGE_TK_DECODER_INFERENCE:
            m->dec_inf.reset(new decoder::InferenceTransformer(
                std::move(q), std::move(k), std::move(v), std::move(pos),
                InferenceMLP(std::move(ffn), std::nullopt), std::move(o), std::move(streams), nt));
            m->dec_inf->block().attention().normalization() = std::move(n1);
            m->dec_inf->block().norm2() = std::move(n2);
            break;
        default: throw Error(FORGE_EINVAL, "unknown transformer kind");
        }
        r.sync();
        *out_model = m.release();
    });
}

extern "C" forge_status forge_net_transformer_forward(forge_net_model* m, forge_slice input,
                                                      forge_slice output) {
    if (!m || (!m->enc_inf && !m->enc_train && !m->dec_inf)) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        const forge_transformer_desc& d = m->desc;
        need(input, d.seq * d.hidden, "transformer input");
        need(output, d.seq * d.out, "transformer output");
        // Input and output are caller buffers: non-owning Matrix views, and
        // the output projection writes straight into the caller's buffer.
        Matrix X(DeviceBuffer(nullptr, forge_slice{input.ptr, d.seq * d.hidden}), d.seq, d.hidden);
        Matrix Y(DeviceBuffer(nullptr, forge_slice{output.ptr, d.seq * d.out}), d.seq, d.out);
        if (m->enc_train) m->enc_train->forward_into(X, Y, rt);
        else if (m->enc_inf) m->enc_inf->forward_into(X, Y, rt);
        else m->dec_inf->forward_into(X, Y, rt);
    });
}

extern "C" forge_status forge_net_transformer_backward(forge_net_model* m, forge_slice dy, float lr,
                                                       forge_slice dx, const forge_slice* grads) {
    if (!m || !m->enc_train) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        const forge_transformer_desc& d = m->desc;
        need(dy, d.seq * d.out, "transformer dy");
        Matrix DY(DeviceBuffer(nullptr, forge_slice{dy.ptr, d.seq * d.out}), d.seq, d.out);
        TransformerGrads g;
        if (present(dx)) {
            // The input gradient goes straight into the caller's buffer.
            need(dx, d.seq * d.hidden, "transformer dx");
            Matrix DX(DeviceBuffer(nullptr, forge_slice{dx.ptr, d.seq * d.hidden}), d.seq,
                      d.hidden);
            m->enc_train->backward_into(DY, lr, rt, DX, grads ? &g : nullptr);
        } else {
            Matrix DX = grads ? m->enc_train->backward_grads(DY, lr, rt, g)
                              : m->enc_train->backward(DY, lr, rt);
        }
        if (grads) {
            const int wslot[6] = {FORGE_TP_WQ, FORGE_TP_WK, FORGE_TP_WV, FORGE_TP_W1, FORGE_TP_W2,
                                  FORGE_TP_WO};
            const int bslot[6] = {FORGE_TP_BQ, FORGE_TP_BK, FORGE_TP_BV, FORGE_TP_B1, FORGE_TP_B2,
                                  FORGE_TP_BO};
            for (int i = 0; i < 6; i++) {
                if (present(grads[wslot[i]])) copy_out(rt, grads[wslot[i]], g.weights[i], "dW");
                if (present(grads[bslot[i]]) && g.biases[i])
                    copy_out(rt, grads[bslot[i]], *g.biases[i], "db");
            }
            if (present(grads[FORGE_TP_POS])) copy_out(rt, grads[FORGE_TP_POS], g.position, "dPos");
            if (present(grads[FORGE_TP_G1]) && g.norm1_gamma)
                copy_out(rt, grads[FORGE_TP_G1], *g.norm1_gamma, "dgamma1");
            if (present(grads[FORGE_TP_BE1]) && g.norm1_beta)
                copy_out(rt, grads[FORGE_TP_BE1], *g.norm1_beta, "dbeta1");
            if (present(grads[FORGE_TP_G2]) && g.norm2_gamma)
                copy_out(rt, grads[FORGE_TP_G2], *g.norm2_gamma, "dgamma2");
            if (present(grads[FORGE_TP_BE2]) && g.norm2_beta)
                copy_out(rt, grads[FORGE_TP_BE2], *g.norm2_beta, "dbeta2");
        }
    });
}

extern "C" forge_status forge_net_transformer_set_score_bytes(forge_net_model* m, size_t bytes) {
    if (!m || (!m->enc_inf && !m->enc_train && !m->dec_inf)) return FORGE_EINVAL;
    return guard([&] { parts_of(m).attention->set_max_score_bytes(bytes); });
}

extern "C" forge_status forge_net_transformer_set_fold_norms(forge_net_model* m, int on) {
    if (!m || (!m->enc_inf && !m->dec_inf)) return FORGE_EINVAL;
    return guard([&] {
        (m->enc_inf ? m->enc_inf->block() : m->dec_inf->block()).set_fold_norms(on != 0);
    });
}

extern "C" forge_status forge_net_transformer_param(forge_net_model* m, int slot,
                                                    forge_slice* out) {
    if (!m || !out || (!m->enc_inf && !m->enc_train && !m->dec_inf)) return FORGE_EINVAL;
    return guard([&] {
        Parts p = parts_of(m);
        QkvProjection& qkv = p.attention->qkv();
        Normalization& n1 = p.attention->normalization();
        switch (slot) {
        case FORGE_TP_WQ: *out = qkv.query().weights().slice(); break;
        case FORGE_TP_BQ: *out = opt(qkv.query().bias()); break;
        case FORGE_TP_WK: *out = qkv.key().weights().slice(); break;
        case FORGE_TP_BK: *out = opt(qkv.key().bias()); break;
        case FORGE_TP_WV: *out = qkv.value().weights().slice(); break;
        case FORGE_TP_BV: *out = opt(qkv.value().bias()); break;
        case FORGE_TP_POS: *out = p.position->slice(); break;
        case FORGE_TP_W1: *out = p.ffn->layers()[0].weights().slice(); break;
        case FORGE_TP_B1: *out = opt(p.ffn->layers()[0].bias()); break;
        case FORGE_TP_W2: *out = p.ffn->layers()[1].weights().slice(); break;
        case FORGE_TP_B2: *out = opt(p.ffn->layers()[1].bias()); break;
        case FORGE_TP_WO: *out = p.output->weights().slice(); break;
        case FORGE_TP_BO: *out = opt(p.output->bias()); break;
        case FORGE_TP_G1: *out = opt(n1.gamma); break;
        case FORGE_TP_BE1: *out = opt(n1.beta); break;
        case FORGE_TP_G2: *out = opt(p.norm2->gamma); break;
        case FORGE_TP_BE2: *out = opt(p.norm2->beta); break;
        default: throw Error(FORGE_EINVAL, "unknown parameter slot");
        }
    });
}

// ============================================================== checkpoint

extern "C" forge_status forge_net_checkpoint_save(forge_net_model* m, const char* path) {
    if (!m || !path) return FORGE_EINVAL;
    return guard([&] {
        CudaRuntime& rt = *m->rt;
        if (m->linear) checkpoint::dump_linear(*m->linear, path, rt);
        else if (m->imlp) checkpoint::dump_inference_mlp(*m->imlp, path, rt);
        else if (m->tmlp) checkpoint::dump_training_mlp(*m->tmlp, path, rt);
        else if (m->enc_inf) checkpoint::dump_transformer(*m->enc_inf, path, rt);
        else if (m->enc_train) checkpoint::dump_training_transformer(*m->enc_train, path, rt);
        else if (m->dec_inf) checkpoint::dump_decoder_transformer(*m->dec_inf, path, rt);
        else throw Error(FORGE_EINVAL, "empty model handle");
    });
}

extern "C" forge_status forge_net_checkpoint_load(forge_runtime* rt, const char* path, int kind,
                                                  forge_net_model** out_model) {
    if (!rt || !path || !out_model) return FORGE_EINVAL;
    *out_model = nullptr;
    return guard([&] {
        std::unique_ptr<forge_net_model> m(new_model(rt));
        CudaRuntime& r = *m->rt;
        switch (kind) {
        case FORGE_CK_LINEAR: m->linear.reset(new Linear(checkpoint::load_linear(path, r))); break;
        case FORGE_CK_MLP_INFERENCE:
            m->imlp.reset(new InferenceMLP(checkpoint::load_inference_mlp(path, r)));
            break;
        case FORGE_CK_MLP_TRAINING:
            m->tmlp.reset(new TrainingMlp(checkpoint::load_training_mlp(path, r)));
            break;
        case FORGE_CK_ENCODER_INFERENCE:
        case FORGE_CK_ENCODER_TRAINING:
        case FORGE_CK_DECODER_INFERENCE: {
            const checkpoint::TransformerMetadata t = checkpoint::read_transformer_metadata(path);
            const size_t hidden = t.position.cols;
            require(t.feed_forward.layers.size() == 2,
                    "a transformer handle needs a two-layer feed-forward network");
            require(t.query.output_neurons == hidden,
                    "a transformer handle needs query/key width equal to the embedding");
            m->desc.seq = t.position.rows;
            m->desc.hidden = hidden;
            m->desc.ffn = t.feed_forward.layers[0].output_neurons;
            m->desc.out = t.output.output_neurons;
            m->desc.norm_type = t.normalization == NormType::Rms ? 0 : 1;
            m->desc.qkv_streams = 0;
            m->desc.ffn_activation = (int)t.feed_forward.layers[0].activation;
            if (kind == FORGE_CK_ENCODER_INFERENCE) {
                m->desc.kind = FORGE_TK_ENCODER_INFERENCE;
                m->enc_inf.reset(
                    new encoder::InferenceTransformer(checkpoint::load_transformer(path, r)));
            } else if (kind == FORGE_CK_ENCODER_TRAINING) {
                m->desc.kind = FORGE_TK_ENCODER_TRAINING;
                m->enc_train.reset(new encoder::TrainingTransformer(
                    checkpoint::load_training_transformer(path, r)));
            } else {
                m->desc.kind = FORGE_TK_DECODER_INFERENCE;
                m->dec_inf.reset(new decoder::InferenceTransformer(
                    checkpoint::load_decoder_transformer(path, r)));
            }
            break;
        }
        default: throw Error(FORGE_EINVAL, "unknown checkpoint kind");
        }
        r.sync();
        *out_model = m.release();
    });
}

extern "C" forge_status forge_checkpoint_inspect(const char* path, char* model_type, size_t cap,
                                                 uint64_t* data_bytes) {
    if (!path) return FORGE_EINVAL;
    return guard([&] {
        uint64_t bytes = 0;
        const std::string type = checkpoint::inspect(path, &bytes);
        if (model_type) {
            require(cap > type.size(), "model_type buffer too small");
            std::memcpy(model_type, type.c_str(), type.size() + 1);
        }
        if (data_bytes) *data_bytes = bytes;
    });
}

extern "C" forge_status forge_net_model_dims(forge_net_model* m, size_t* dims, size_t cap,
                                             size_t* count) {
    if (!m || !count || (cap && !dims)) return FORGE_EINVAL;
    return guard([&] {
        std::vector<size_t> d;
        if (m->linear) {
            d = {m->linear->weights().rows(), m->linear->weights().cols()};
        } else if (m->imlp || m->tmlp) {
            MlpExecutor& ex = mlp_exec(m);
            d.push_back(ex.layers().front().weights().rows());
            for (const Linear& l : ex.layers()) d.push_back(l.weights().cols());
        } else if (m->enc_inf || m->enc_train || m->dec_inf) {
            d = {m->desc.seq, m->desc.hidden, m->desc.ffn, m->desc.out};
        } else {
            throw Error(FORGE_EINVAL, "empty model handle");
        }
        *count = d.size();
        for (size_t i = 0; i < d.size() && i < cap; i++) dims[i] = d[i];
    });
}

extern "C" forge_status forge_net_transformer_describe(forge_net_model* m,
                                                       forge_transformer_desc* out) {
    if (!m || !out || (!m->enc_inf && !m->enc_train && !m->dec_inf)) return FORGE_EINVAL;
    *out = m->desc;
    return FORGE_OK;
}
