// executors.cpp -- Linear, MLP, Attention and the single-head Post-Norm
// transformer blocks (reference src/net/linear.rs, mlp.rs,
// transformer/{attention,inference,encoder,decoder}.rs).
//
// The arithmetic order of every fused step matches the reference's separate
// launches (each fused operation is one rounded f32 op in the same order, and
// a+b == b+a exactly), so the fused executors compute what the reference's
// launch sequence computes on the same GEMM products.
#include <cmath>

#include "oxforge_net.hpp"

namespace oxforge {

static void require(bool cond, const char* what) {
    if (!cond) throw Error(FORGE_EINVAL, std::string("assertion failed: ") + what);
}

static forge_map_op forward_map(Activation a) {
    switch (a) {
    case Activation::Gelu: return FORGE_MAP_GELU;
    case Activation::Relu: return FORGE_MAP_RELU;
    case Activation::Silu: return FORGE_MAP_SILU;
    default: return FORGE_MAP_IDENTITY;
    }
}

// SGD on a parameter vector, as Linear::learn updates a bias
// (linear.rs:385-390): scaled = clone(grad) * lr; param -= scaled, as one
// kernel with the same two roundings.
static void sgd_vector(CudaRuntime& rt, Vector& param, const Vector& grad, float lr,
                       const CudaStream* stream = nullptr) {
    require(param.len() == grad.len(), "parameter and gradient lengths");
    check(forge_sgd_update(rt.raw(), stream_raw(stream), param.slice(), grad.slice(), param.len(),
                           lr),
          "sgd_update");
}

// Norm backward for a training step: computes dgamma/dbeta whenever the norm
// has parameters (to update them) or gradients are requested, applies SGD to
// the norm's own gamma/beta, and hands the gradients to the caller.
static Matrix norm_backward_step(Normalization& norm, const Matrix& input,
                                 const Matrix& output_gradient, float lr, CudaRuntime& rt,
                                 bool want, std::optional<Vector>* out_gamma,
                                 std::optional<Vector>* out_beta, const Matrix* dot_sub = nullptr,
                                 Vector* dot = nullptr, float dot_scale = 1.0f) {
    const size_t cols = input.cols();
    std::optional<Vector> dg, db;
    if (want) dg = Vector(rt.get_uninit_buffer(cols));
    if (norm.kind == NormType::Layer && want) db = Vector(rt.get_uninit_buffer(cols));
    Matrix dx = norm.backward_step(input, output_gradient, lr, rt, dg ? &*dg : nullptr,
                                   db ? &*db : nullptr, dot_sub, dot, dot_scale);
    if (want) {
        *out_gamma = std::move(dg);
        *out_beta = std::move(db);
    }
    return dx;
}

// ================================================================== Linear

Linear::Linear(Matrix weights, std::optional<Vector> bias, Activation activation)
    : weights_(std::move(weights)), bias_(std::move(bias)), activation_(activation) {
    if (bias_) require(bias_->len() == weights_.cols(), "bias.len() == weights.cols()");
}

LinearMetadata Linear::get_meta_data(MetadataCursor& cursor) const {
    // linear.rs:97-105.
    LinearMetadata m;
    m.input_neurons = weights_.rows();
    m.output_neurons = weights_.cols();
    m.activation = activation_;
    m.weights = cursor.matrix(weights_.rows(), weights_.cols());
    if (bias_) m.bias = cursor.vector(bias_->len());
    return m;
}

std::vector<HostData> Linear::get_data(CudaRuntime& rt) const {
    // linear.rs:107-114.
    std::vector<HostData> data;
    data.reserve(bias_ ? 2 : 1);
    data.emplace_back(weights_.to_host(rt));
    if (bias_) data.emplace_back(bias_->to_host(rt));
    return data;
}

Matrix Linear::forward_keep(const Matrix& input, const Matrix* residual, Matrix* pre_activation,
                            CudaRuntime& rt, const CudaStream* stream) {
    // linear.rs:116-132 -> affine_on (185-206) + activate_on (225-230).
    require(input.cols() == weights_.rows(), "input.cols() == weights.rows()");
    Matrix out = rt.new_uninit_matrix(input.rows(), weights_.cols());
    forward_into(input, residual, out, rt, stream, pre_activation);
    return out;
}

void Linear::forward_into(const Matrix& input, const Matrix* residual, Matrix& out,
                          CudaRuntime& rt, const CudaStream* stream, Matrix* pre_activation) {
    require(input.cols() == weights_.rows(), "input.cols() == weights.rows()");
    require(out.rows() == input.rows() && out.cols() == weights_.cols(), "output shape");
    rt.stream_join_primary(stream);
    forge_gemm_epilogue ep = plain_epilogue();
    if (bias_) ep.bias = bias_->slice();
    if (residual) {
        require(residual->rows() == out.rows() && residual->cols() == out.cols(),
                "residual shape");
        ep.residual = residual->slice();
    }
    if (pre_activation) {
        require(pre_activation->rows() == out.rows() && pre_activation->cols() == out.cols(),
                "pre-activation shape");
        ep.pre_out = pre_activation->slice();
    }
    ep.activation = (int)activation_;
    rt.gemm_ex(stream, false, false, input, weights_, out.slice(), input.rows(), weights_.cols(),
               input.cols(), ep);
}

forge_gemm_problem Linear::forward_problem(const Matrix& input, Matrix& out) const {
    require(input.cols() == weights_.rows(), "input.cols() == weights.rows()");
    require(out.rows() == input.rows() && out.cols() == weights_.cols(), "output shape");
    forge_gemm_problem pr{};
    pr.A = input.slice();
    pr.B = weights_.slice();
    pr.C = out.slice();
    pr.epilogue = plain_epilogue();
    if (bias_) pr.epilogue.bias = bias_->slice();
    pr.epilogue.activation = (int)activation_;
    return pr;
}

Matrix Linear::forward(const Matrix& input, const Matrix* residual, CudaRuntime& rt,
                       const CudaStream* stream) {
    return forward_keep(input, residual, nullptr, rt, stream);
}

Matrix Linear::affine(const Matrix& input, const Matrix* residual, CudaRuntime& rt,
                      const CudaStream* stream) {
    // linear.rs:157-206: product, bias by rows, residual; no activation.
    require(input.cols() == weights_.rows(), "input.cols() == weights.rows()");
    Matrix out = rt.new_uninit_matrix(input.rows(), weights_.cols());
    rt.stream_join_primary(stream);
    forge_gemm_epilogue ep = plain_epilogue();
    if (bias_) ep.bias = bias_->slice();
    if (residual) {
        require(residual->rows() == out.rows() && residual->cols() == out.cols(),
                "residual shape");
        ep.residual = residual->slice();
    }
    rt.gemm_ex(stream, false, false, input, weights_, out.slice(), input.rows(), weights_.cols(),
               input.cols(), ep);
    return out;
}

void Linear::activate(Matrix& output, CudaRuntime& rt, const CudaStream* stream) {
    // linear.rs:208-230.
    if (activation_ != Activation::Identity) output.map(forward_map(activation_), 0.0f, rt, stream);
}

std::pair<Matrix, std::optional<Vector>> Linear::backward(const Matrix* pre_activation,
                                                          const Matrix& output_gradient,
                                                          CudaRuntime& rt,
                                                          const CudaStream* stream) {
    // linear.rs:232-306: gradient = dY * act'(pre); bias gradient = column
    // sums (the reference's transpose + sum_rows).
    Matrix gradient = rt.new_uninit_matrix(output_gradient.rows(), output_gradient.cols());
    rt.stream_join_primary(stream);
    if (activation_ != Activation::Identity) {
        require(pre_activation != nullptr, "activation backward requires pre-activation");
        require(pre_activation->rows() == output_gradient.rows() &&
                    pre_activation->cols() == output_gradient.cols(),
                "pre-activation shape");
        check(forge_activation_backward(rt.raw(), stream_raw(stream), output_gradient.slice(),
                                        pre_activation->slice(), gradient.slice(), gradient.len(),
                                        (forge_activation)activation_),
              "Linear::backward");
    } else {
        check(forge_memcpy_d2d(rt.raw(), stream_raw(stream), gradient.slice(), output_gradient.slice(),
                               gradient.len()),
              "Linear::backward");
    }
    std::optional<Vector> bias_gradient;
    if (bias_) bias_gradient = rt.matrix_sum_cols(gradient, stream);
    return {std::move(gradient), std::move(bias_gradient)};
}

Vector Linear::loss_rows(const Matrix& output, const Matrix& target, CudaRuntime& rt,
                         const CudaStream* stream) {
    // linear.rs:312-348: mean over columns of 0.5 * (o - t)^2 per row.
    Matrix loss = rt.matrix_binary_on(stream, output, target, BinaryOp::Sub);
    loss.map(FORGE_MAP_HALF_SQ, 0.0f, rt, stream);
    float cols = (float)loss.cols();
    Vector row_loss = rt.matrix_sum_rows_on(loss, stream);
    row_loss.scale_on(1.0f / cols, rt, stream);
    return row_loss;
}

forge_gemm_problem Linear::learn_problem(const Matrix& input, const Matrix& gradient,
                                         float learning_rate, Matrix* weight_gradient) {
    require(input.rows() == gradient.rows(), "input.rows() == gradient.rows()");
    require(input.cols() == weights_.rows() && gradient.cols() == weights_.cols(),
            "learn shapes");
    forge_gemm_problem pr{};
    pr.A = input.slice();
    pr.B = gradient.slice();
    pr.C = weights_.slice();
    pr.epilogue = plain_epilogue();
    pr.epilogue.update = 1;
    pr.epilogue.update_scale = learning_rate;
    if (weight_gradient) {
        require(weight_gradient->rows() == weights_.rows() &&
                    weight_gradient->cols() == weights_.cols(),
                "weight gradient shape");
        pr.epilogue.pre_out = weight_gradient->slice();
    }
    return pr;
}

void Linear::learn_keep(const Matrix& input, const Matrix& gradient, const Vector* bias_gradient,
                        float learning_rate, Matrix* weight_gradient, CudaRuntime& rt,
                        const CudaStream* stream, bool bias_step) {
    // linear.rs:373-415: W -= lr * (X^T G) as one TN GEMM whose epilogue
    // scales by lr and subtracts from W; b -= lr * db.
    require(input.rows() == gradient.rows(), "input.rows() == gradient.rows()");
    require(input.cols() == weights_.rows() && gradient.cols() == weights_.cols(),
            "learn shapes");
    rt.stream_join_primary(stream);
    forge_gemm_epilogue ep = plain_epilogue();
    ep.update = 1;
    ep.update_scale = learning_rate;
    if (weight_gradient) {
        require(weight_gradient->rows() == weights_.rows() &&
                    weight_gradient->cols() == weights_.cols(),
                "weight gradient shape");
        ep.pre_out = weight_gradient->slice();
    }
    rt.gemm_ex(stream, true, false, input, gradient, weights_.slice(), weights_.rows(),
               weights_.cols(), input.rows(), ep);
    if (bias_ && bias_step) {
        require(bias_gradient != nullptr, "missing bias gradient for biased Linear");
        sgd_vector(rt, *bias_, *bias_gradient, learning_rate, stream);
    }
}

void Linear::learn_from_gradient(const Matrix& input, const Matrix& gradient,
                                 float learning_rate, Matrix* weight_gradient,
                                 std::optional<Vector>* bias_gradient_out, CudaRuntime& rt,
                                 const CudaStream* stream) {
    learn_keep(input, gradient, nullptr, learning_rate, weight_gradient, rt, stream,
               /*bias_step=*/false);
    if (!bias_) return;
    forge_slice out{nullptr, 0};
    if (bias_gradient_out) {
        *bias_gradient_out = Vector(rt.get_uninit_buffer(gradient.cols()));
        out = (*bias_gradient_out)->slice();
    }
    check(forge_sum_cols_sgd(rt.raw(), stream_raw(stream), gradient.slice(), gradient.rows(),
                             gradient.cols(), out, bias_->slice(), learning_rate),
          "bias gradient and update");
}

void Linear::learn(const Matrix& input, const Matrix& gradient, const Vector* bias_gradient,
                   float learning_rate, CudaRuntime& rt, const CudaStream* stream) {
    learn_keep(input, gradient, bias_gradient, learning_rate, nullptr, rt, stream);
}

Matrix Linear::input_gradient(const Matrix& gradient, CudaRuntime& rt, const CudaStream* stream) {
    // linear.rs:417-444: G * W^T as an NT GEMM (no materialised W^T).
    require(gradient.cols() == weights_.cols(), "gradient.cols() == weights.cols()");
    Matrix out = rt.new_uninit_matrix(gradient.rows(), weights_.rows());
    rt.stream_join_primary(stream);
    rt.gemm_ex(stream, false, true, gradient, weights_, out.slice(), gradient.rows(),
               weights_.rows(), weights_.cols(), plain_epilogue());
    return out;
}

void Linear::input_gradient_accumulate(const Matrix& gradient, Matrix& accumulate,
                                       CudaRuntime& rt, const CudaStream* stream) {
    require(gradient.cols() == weights_.cols(), "gradient.cols() == weights.cols()");
    require(accumulate.rows() == gradient.rows() && accumulate.cols() == weights_.rows(),
            "accumulator shape");
    rt.stream_join_primary(stream);
    forge_gemm_epilogue ep = plain_epilogue();
    ep.residual = accumulate.slice();
    rt.gemm_ex(stream, false, true, gradient, weights_, accumulate.slice(), gradient.rows(),
               weights_.rows(), weights_.cols(), ep);
}

std::pair<Matrix, std::optional<Vector>> Linear::backward_with_res(
    const Matrix& pre_activation, const Matrix& output_gradient, const Matrix& residual_gradient,
    CudaRuntime& rt, const CudaStream* stream) {
    // linear.rs:446-532: (dY + dR) * act'(pre), bias gradient.
    require(pre_activation.rows() == output_gradient.rows() &&
                pre_activation.cols() == output_gradient.cols(),
            "pre-activation shape");
    require(output_gradient.rows() == residual_gradient.rows() &&
                output_gradient.cols() == residual_gradient.cols(),
            "residual gradient shape");
    Matrix sum = rt.matrix_binary_on(stream, output_gradient, residual_gradient, BinaryOp::Add);
    Matrix gradient = rt.new_uninit_matrix(sum.rows(), sum.cols());
    if (activation_ != Activation::Identity) {
        check(forge_activation_backward(rt.raw(), stream_raw(stream), sum.slice(), pre_activation.slice(),
                                        gradient.slice(), gradient.len(),
                                        (forge_activation)activation_),
              "backward_with_res");
    } else {
        gradient = std::move(sum);
    }
    std::optional<Vector> bias_gradient;
    if (bias_) bias_gradient = rt.matrix_sum_cols(gradient, stream);
    return {std::move(gradient), std::move(bias_gradient)};
}

// ===================================================================== MLP

MlpExecutor::MlpExecutor(std::vector<Linear> layers,
                         std::optional<std::pair<size_t, size_t>> res_range, Loss loss)
    : layers_(std::move(layers)), res_range_(res_range), loss_(loss) {
    require(!layers_.empty(), "MLP must contain at least one layer");
    if (res_range_)
        require(res_range_->first < res_range_->second && res_range_->second <= layers_.size(),
                "invalid residual range");
}

MlpMetadata MlpExecutor::get_meta_data(MetadataCursor& cursor) const {
    // mlp.rs:99-112.
    MlpMetadata m;
    m.layer_count = layers_.size();
    m.loss = loss_;
    if (res_range_) m.residual = ResidualMetadata{res_range_->first, res_range_->second};
    for (const Linear& l : layers_) m.layers.push_back(l.get_meta_data(cursor));
    return m;
}

std::vector<HostData> MlpExecutor::get_data(CudaRuntime& rt) const {
    // mlp.rs:114-119.
    std::vector<HostData> data;
    for (const Linear& l : layers_)
        for (HostData& d : l.get_data(rt)) data.push_back(std::move(d));
    return data;
}

Matrix MlpExecutor::forward(const Matrix& input, CudaRuntime& rt) {
    return forward_plus(input, nullptr, rt);
}

Matrix MlpExecutor::forward_plus(const Matrix& input, const Matrix* final_residual,
                                 CudaRuntime& rt) {
    // mlp.rs:53-85.  The residual source is kept alive instead of cloned.
    const size_t L = layers_.size();
    std::vector<std::optional<Matrix>> outs(L);
    auto in_of = [&](size_t i) -> const Matrix& { return i == 0 ? input : *outs[i - 1]; };
    for (size_t i = 0; i < L; i++) {
        const bool consumes = res_range_ && i + 1 == res_range_->second;
        const Matrix* residual = consumes ? &in_of(res_range_->first) : nullptr;
        const Matrix* extra = i + 1 == L ? final_residual : nullptr;
        Matrix out;
        if (residual && extra) {
            out = layers_[i].forward(in_of(i), residual, rt, nullptr);
            out.binary_assign(*extra, BinaryOp::Add, rt);
        } else {
            out = layers_[i].forward(in_of(i), residual ? residual : extra, rt, nullptr);
        }
        outs[i] = std::move(out);
        if (i >= 1) {
            const size_t k = i - 1;  // outs[k] was the input of layer i
            const bool keep = res_range_ && res_range_->first == i && i + 1 < res_range_->second;
            if (!keep) outs[k].reset();
        }
        if (consumes && res_range_->first >= 1) outs[res_range_->first - 1].reset();
    }
    return std::move(*outs[L - 1]);
}

Matrix MlpExecutor::backward(const std::vector<Matrix>& layer_inputs,
                             const std::vector<Matrix>& pre_activations,
                             const Matrix& output_gradient, float learning_rate, CudaRuntime& rt,
                             std::vector<Matrix>* weight_gradients,
                             std::vector<std::optional<Vector>>* bias_gradients,
                             const Matrix* input_gradient_residual) {
    // mlp.rs:121-168, last layer first.  When the previous layer has a cached
    // pre-activation and no residual gradient joins at this boundary, its
    // act'(z) multiply is fused into this layer's input-gradient GEMM.
    const size_t L = layers_.size();
    require(layer_inputs.size() == L, "layer_inputs.len() == layers.len()");
    if (weight_gradients) weight_gradients->resize(L);
    if (bias_gradients) bias_gradients->resize(L);
    auto cached_pre = [&](size_t i) -> const Matrix* {
        return i < pre_activations.size() && pre_activations[i].len() ? &pre_activations[i]
                                                                       : nullptr;
    };
    const Matrix* grad = &output_gradient;
    std::optional<Matrix> grad_owned;
    bool grad_preactivated = false;
    std::optional<std::pair<size_t, Matrix>> residual_gradient;
    // A layer whose G was formed in the next layer's input-gradient epilogue
    // may also have had its bias gradient and SGD step taken there (from the
    // epilogue's column sums): bias_done, with the sums in carried_bias.
    bool bias_done = false;
    std::optional<Vector> carried_bias;

    for (size_t step = 0; step < L; step++) {
        const size_t index = L - 1 - step;
        Linear& layer = layers_[index];
        std::optional<size_t> residual_index;
        if (res_range_ && index + 1 == res_range_->second) residual_index = res_range_->first;

        // Layer gradient: dY * act'(pre).
        std::optional<Matrix> layer_grad_owned;
        std::optional<Vector> bias_gradient = std::move(carried_bias);
        const bool this_bias_done = bias_done;
        carried_bias.reset();
        bias_done = false;
        const Matrix* layer_gradient = grad;
        if (layer.needs_pre_activation() && !grad_preactivated) {
            const Matrix* pre = cached_pre(index);
            std::optional<Matrix> recomputed;
            if (!pre) {
                const Matrix* residual =
                    residual_index ? &layer_inputs[*residual_index] : nullptr;
                recomputed = layer.affine(layer_inputs[index], residual, rt, nullptr);
                pre = &*recomputed;
            }
            auto gb = layer.backward(pre, *grad, rt, nullptr);
            layer_grad_owned = std::move(gb.first);
            bias_gradient = std::move(gb.second);
            layer_gradient = &*layer_grad_owned;
        }
        // The bias gradient of a layer whose G arrived pre-multiplied is formed
        // at the update, with the bias's SGD step (learn_from_gradient),
        // unless the previous GEMM's epilogue took it already.
        const bool defer_bias = layer.bias() && !bias_gradient && !this_bias_done;

        // Input gradient G * W^T (+ act' of the previous layer, fused).
        const bool skip_now = (residual_index && *residual_index == index) ||
                              (residual_gradient && residual_gradient->first == index);
        Linear* prev = index > 0 ? &layers_[index - 1] : nullptr;
        const Matrix* prev_pre = index > 0 ? cached_pre(index - 1) : nullptr;
        const bool fuse_prev = prev && prev->needs_pre_activation() && prev_pre && !skip_now;
        const bool add_external = index == 0 && input_gradient_residual;
        Matrix input_gradient = rt.new_uninit_matrix(layer_gradient->rows(), layer.weights().rows());
        forge_gemm_epilogue ep = plain_epilogue();
        if (fuse_prev) {
            ep.aux_mul = prev_pre->slice();
            ep.aux_activation = (int)prev->activation();
        }
        if (add_external && !skip_now) {
            require(input_gradient_residual->rows() == input_gradient.rows() &&
                        input_gradient_residual->cols() == input_gradient.cols(),
                    "input gradient residual shape");
            ep.residual = input_gradient_residual->slice();
        }
        // The epilogue's output is then exactly the previous layer's G: its
        // column sums are that layer's bias gradient (linear.rs:267-272), and
        // the bias takes its SGD step (linear.rs:385-390) in the same pass.
        if (fuse_prev && prev->bias() && !ep.residual.ptr) {
            if (bias_gradients) {
                carried_bias = Vector(rt.get_uninit_buffer(prev->bias()->len()));
                ep.col_sums_out = carried_bias->slice();
            }
            ep.col_sums_param = prev->bias()->slice();
            ep.col_sums_lr = learning_rate;
            bias_done = true;
        }
        rt.gemm_ex(nullptr, false, true, *layer_gradient, layer.weights(), input_gradient.slice(),
                   layer_gradient->rows(), layer.weights().rows(), layer.weights().cols(), ep);

        if (residual_index)
            residual_gradient = std::make_pair(*residual_index, rt.clone_matrix(*layer_gradient));
        if (residual_gradient && residual_gradient->first == index) {
            input_gradient.binary_assign(residual_gradient->second, BinaryOp::Add, rt);
            residual_gradient.reset();
        }
        if (add_external && skip_now)
            input_gradient.binary_assign(*input_gradient_residual, BinaryOp::Add, rt);

        Matrix* wg = nullptr;
        if (weight_gradients) {
            (*weight_gradients)[index] =
                rt.new_uninit_matrix(layer.weights().rows(), layer.weights().cols());
            wg = &(*weight_gradients)[index];
        }
        if (defer_bias) {
            layer.learn_from_gradient(layer_inputs[index], *layer_gradient, learning_rate, wg,
                                      bias_gradients ? &bias_gradient : nullptr, rt, nullptr);
        } else {
            layer.learn_keep(layer_inputs[index], *layer_gradient,
                             bias_gradient ? &*bias_gradient : nullptr, learning_rate, wg, rt,
                             nullptr, /*bias_step=*/!this_bias_done);
        }
        if (bias_gradients) (*bias_gradients)[index] = std::move(bias_gradient);

        grad_owned = std::move(input_gradient);
        grad = &*grad_owned;
        grad_preactivated = fuse_prev;
    }
    require(!residual_gradient, "unresolved residual gradient");
    return std::move(*grad_owned);
}

Matrix TrainingMlp::forward(Matrix input, CudaRuntime& rt) {
    return forward_plus(std::move(input), false, rt);
}

Matrix TrainingMlp::forward_plus(Matrix input, bool add_input_to_output, CudaRuntime& rt) {
    // mlp.rs:233-254; the pre-activation of every activated layer is kept.
    auto& layers = executor_.layers();
    const size_t L = layers.size();
    const auto res = executor_.res_range();
    layer_inputs_.clear();
    pre_activations_.clear();
    layer_inputs_.reserve(L);
    pre_activations_.resize(L);
    layer_inputs_.push_back(std::move(input));
    for (size_t i = 0; i < L; i++) {
        const Matrix* residual = (res && i + 1 == res->second) ? &layer_inputs_[res->first] : nullptr;
        const Matrix* extra = (i + 1 == L && add_input_to_output) ? &layer_inputs_[0] : nullptr;
        Matrix* pre = nullptr;
        if (layers[i].needs_pre_activation()) {
            pre_activations_[i] = rt.new_uninit_matrix(layer_inputs_[i].rows(), layers[i].weights().cols());
            pre = &pre_activations_[i];
        }
        Matrix out;
        if (residual && extra) {
            out = layers[i].forward_keep(layer_inputs_[i], residual, pre, rt, nullptr);
            out.binary_assign(*extra, BinaryOp::Add, rt);
        } else {
            out = layers[i].forward_keep(layer_inputs_[i], residual ? residual : extra, pre, rt,
                                         nullptr);
        }
        if (i + 1 == L) return out;
        layer_inputs_.push_back(std::move(out));
    }
    throw Error(FORGE_EINVAL, "MLP always contains at least one layer");
}

Matrix TrainingMlp::backward(const Matrix& output_gradient, float learning_rate, CudaRuntime& rt) {
    return executor_.backward(layer_inputs_, pre_activations_, output_gradient, learning_rate, rt);
}

Matrix TrainingMlp::backward_grads(const Matrix& output_gradient, float learning_rate,
                                   CudaRuntime& rt, std::vector<Matrix>* weight_gradients,
                                   std::vector<std::optional<Vector>>* bias_gradients,
                                   const Matrix* input_gradient_residual) {
    return executor_.backward(layer_inputs_, pre_activations_, output_gradient, learning_rate, rt,
                              weight_gradients, bias_gradients, input_gradient_residual);
}

// =========================================================== Normalization

void Normalization::forward(Matrix& m, CudaRuntime& rt) const { forward_into(m, m, rt); }

void Normalization::forward_into(const Matrix& src, Matrix& dst, CudaRuntime& rt) const {
    require(src.rows() == dst.rows() && src.cols() == dst.cols(), "norm output shape");
    if (src.rows() == 0) return;
    if (kind == NormType::Layer)
        check(forge_layer_norm_rows_out(rt.raw(), nullptr, src.slice(), dst.slice(),
                                        gamma ? gamma->slice() : forge_slice{nullptr, 0},
                                        beta ? beta->slice() : forge_slice{nullptr, 0},
                                        src.rows(), src.cols(), eps),
              "layer_norm");
    else
        check(forge_rms_norm_rows_out(rt.raw(), nullptr, src.slice(), dst.slice(),
                                      gamma ? gamma->slice() : forge_slice{nullptr, 0},
                                      src.rows(), src.cols(), eps),
              "rms_norm");
}

Matrix Normalization::backward(const Matrix& input, const Matrix& output_gradient,
                               CudaRuntime& rt, Vector* dgamma, Vector* dbeta) const {
    require(input.rows() == output_gradient.rows() && input.cols() == output_gradient.cols(),
            "norm backward shapes");
    Matrix out = rt.new_uninit_matrix(input.rows(), input.cols());
    forge_slice g = gamma ? gamma->slice() : forge_slice{nullptr, 0};
    forge_slice dg = dgamma ? dgamma->slice() : forge_slice{nullptr, 0};
    forge_slice db = dbeta ? dbeta->slice() : forge_slice{nullptr, 0};
    if (kind == NormType::Layer)
        check(forge_layer_norm_bwd(rt.raw(), nullptr, input.slice(), output_gradient.slice(), g,
                                   out.slice(), dg, db, input.rows(), input.cols(), eps),
              "layer_norm_backward");
    else
        check(forge_rms_norm_bwd(rt.raw(), nullptr, input.slice(), output_gradient.slice(), g,
                                 out.slice(), dg, input.rows(), input.cols(), eps),
              "rms_norm_backward");
    return out;
}

Matrix Normalization::backward_step(const Matrix& input, const Matrix& output_gradient,
                                    float learning_rate, CudaRuntime& rt, Vector* dgamma,
                                    Vector* dbeta, const Matrix* dot_sub, Vector* dot,
                                    float dot_scale) {
    require(input.rows() == output_gradient.rows() && input.cols() == output_gradient.cols(),
            "norm backward shapes");
    require(!dot_sub == !dot, "row dot needs both dot_sub and dot");
    if (dot_sub)
        require(dot_sub->rows() == input.rows() && dot_sub->cols() == input.cols() &&
                    dot->len() == input.rows(),
                "row dot shapes");
    Matrix out = rt.new_uninit_matrix(input.rows(), input.cols());
    forge_slice g = gamma ? gamma->slice() : forge_slice{nullptr, 0};
    forge_slice b = beta ? beta->slice() : forge_slice{nullptr, 0};
    forge_slice dg = dgamma ? dgamma->slice() : forge_slice{nullptr, 0};
    forge_slice db = dbeta ? dbeta->slice() : forge_slice{nullptr, 0};
    const size_t rows = input.rows(), cols = input.cols();
    if (kind == NormType::Layer && dot_sub)
        check(forge_layer_norm_bwd_sgd_dot(rt.raw(), nullptr, input.slice(),
                                           output_gradient.slice(), g, b, out.slice(), dg, db,
                                           dot_sub->slice(), dot->slice(), rows, cols, eps,
                                           learning_rate, dot_scale),
              "layer_norm_backward");
    else if (kind == NormType::Layer)
        check(forge_layer_norm_bwd_sgd(rt.raw(), nullptr, input.slice(), output_gradient.slice(), g,
                                       b, out.slice(), dg, db, rows, cols, eps, learning_rate),
              "layer_norm_backward");
    else if (dot_sub)
        check(forge_rms_norm_bwd_sgd_dot(rt.raw(), nullptr, input.slice(),
                                         output_gradient.slice(), g, out.slice(), dg,
                                         dot_sub->slice(), dot->slice(), rows, cols, eps,
                                         learning_rate, dot_scale),
              "rms_norm_backward");
    else
        check(forge_rms_norm_bwd_sgd(rt.raw(), nullptr, input.slice(), output_gradient.slice(), g,
                                     out.slice(), dg, rows, cols, eps, learning_rate),
              "rms_norm_backward");
    return out;
}

// ======================================================== QkvProjection

QkvProjection::QkvProjection(Linear query, Linear key, Linear value,
                             std::optional<std::vector<CudaStream>> streams)
    : query_(std::move(query)), key_(std::move(key)), value_(std::move(value)),
      streams_(std::move(streams)) {
    if (streams_) require(streams_->size() == 3, "Q/K/V execution requires three streams");
}

QkvProjection::Projected QkvProjection::project(const Matrix& query_input,
                                                const Matrix& key_value_input, CudaRuntime& rt) {
    Projected p;
    Linear* lins[3] = {&query_, &key_, &value_};
    const Matrix* ins[3] = {&query_input, &key_value_input, &key_value_input};
    Matrix* outs[3] = {&p.query, &p.key, &p.value};
    bool same = true;
    for (int z = 0; z < 3; z++) {
        require(ins[z]->cols() == lins[z]->weights().rows(), "input.cols() == weights.rows()");
        *outs[z] = rt.new_uninit_matrix(ins[z]->rows(), lins[z]->weights().cols());
        same = same && ins[z]->rows() == ins[0]->rows() && ins[z]->cols() == ins[0]->cols() &&
               outs[z]->cols() == outs[0]->cols();
    }
    if (streams_) {
        // attention.rs:65-94: the extra streams wait for the primary stream,
        // then Linear::forward of Q, K and V on streams 0, 1 and 2.
        wait_for_query_key(rt);
        wait_for_value(rt);
        rt.fork_streams(*streams_);
        for (int z = 0; z < 3; z++)
            lins[z]->forward_into(*ins[z], nullptr, *outs[z], rt, &(*streams_)[z]);
        joined_qk_ = joined_v_ = false;
    } else if (same) {
        forge_gemm_problem probs[3];
        for (int z = 0; z < 3; z++) probs[z] = lins[z]->forward_problem(*ins[z], *outs[z]);
        check(forge_gemm_batch_f32(rt.raw(), nullptr, 0, 0, ins[0]->rows(), outs[0]->cols(),
                                   ins[0]->cols(), 3, probs),
              "qkv projection");
    } else {
        for (int z = 0; z < 3; z++) lins[z]->forward_into(*ins[z], nullptr, *outs[z], rt, nullptr);
    }
    return p;
}

// attention.rs:96-102: the primary stream waits for the Q and K streams,
// then for the V stream.  Nothing to wait for when the projections ran on
// the primary stream.
void QkvProjection::wait_for_query_key(CudaRuntime& rt) {
    if (joined_qk_) return;
    rt.join_streams({(*streams_)[0], (*streams_)[1]});
    joined_qk_ = true;
}

void QkvProjection::wait_for_value(CudaRuntime& rt) {
    if (joined_v_) return;
    rt.join_streams({(*streams_)[2]});
    joined_v_ = true;
}

// ============================================================== Attention

Attention::Attention(Linear query, Linear key, Linear value,
                     std::optional<std::vector<CudaStream>> streams, Normalization norm)
    : qkv_(std::move(query), std::move(key), std::move(value), std::move(streams)),
      norm_(std::move(norm)) {}

void Attention::normalize(Matrix& m, CudaRuntime& rt, const Normalization* norm) const {
    (norm ? *norm : norm_).forward(m, rt);
}

static float score_scale(size_t query_cols) {
    // attention.rs:372,398: 1.0 / (query.cols as f32).sqrt()
    return 1.0f / std::sqrt((float)query_cols);
}

// Query rows per score chunk: all of them while S x Sk floats fit the
// budget, else the largest multiple of 64 rows that does (at least 64).
static size_t score_chunk_rows(size_t S, size_t Sk, size_t budget_bytes) {
    const size_t row_bytes = Sk * sizeof(float);
    if (row_bytes == 0 || S <= budget_bytes / row_bytes) return S;
    return std::max<size_t>(64, budget_bytes / row_bytes / 64 * 64);
}

// Rows r0 .. r0 + n - 1 of a row-major matrix as a slice.
static forge_slice rows_of(const Matrix& m, size_t r0, size_t n) {
    return forge_slice{m.buffer().ptr() + r0 * m.cols(), n * m.cols()};
}

static void gemm_slices(CudaRuntime& rt, bool ta, bool tb, forge_slice a, forge_slice b,
                        forge_slice c, size_t m, size_t n, size_t k,
                        const forge_gemm_epilogue& ep, const char* what) {
    check(forge_gemm_ex_f32(rt.raw(), nullptr, ta ? 1 : 0, tb ? 1 : 0, a, b, c, m, n, k, &ep),
          what);
}

void Attention::chunked_forward(const Matrix& q, const Matrix& k, const Matrix& v,
                                const Matrix& residual, bool mask, size_t chunk, Matrix& out,
                                CudaRuntime& rt, Matrix* row_sumsq) {
    // attention.rs:359-387 one chunk of query rows at a time: the chunk's
    // scores (NT GEMM, scale fused), mask, softmax, then its rows of
    // P V + residual.  Each output row is the same sum as in the unchunked
    // products while neither product is computed as K slices; a chunk's
    // P V has few tiles and may be split over Sk (Sk >= 2048, see
    // choose_splits) where the whole product is not, and then the rows agree
    // to within rounding.
    const size_t S = q.rows(), Sk = k.rows(), D = q.cols(), H = v.cols();
    Matrix scores = rt.new_uninit_matrix(std::min(chunk, S), Sk);
    forge_gemm_epilogue ep = plain_epilogue();
    ep.alpha = score_scale(D);
    for (size_t r0 = 0; r0 < S; r0 += chunk) {
        const size_t n = std::min(chunk, S - r0);
        const forge_slice sc{scores.buffer().ptr(), n * Sk};
        gemm_slices(rt, false, true, rows_of(q, r0, n), k.slice(), sc, n, Sk, D, ep,
                    "attention scores");
        if (mask)
            check(forge_causal_mask_rows(rt.raw(), nullptr, sc, n, Sk, r0), "causal_mask");
        check(forge_softmax_rows(rt.raw(), nullptr, sc, n, Sk), "softmax_rows");
        forge_gemm_epilogue ep2 = plain_epilogue();
        ep2.residual = rows_of(residual, r0, n);
        if (row_sumsq) ep2.row_sumsq_out = rows_of(*row_sumsq, r0, n);
        gemm_slices(rt, false, false, sc, v.slice(), rows_of(out, r0, n), n, H, Sk, ep2,
                    "attention value");
    }
}

Matrix Attention::attention_value(QkvProjection::Projected projected, const Matrix& residual,
                                  bool mask, CudaRuntime& rt, Matrix* row_sumsq) {
    // attention.rs:336-387: S = Q K^T / sqrt(d) as one NT GEMM with the
    // scale in its epilogue; (mask); softmax; A = P V with the residual add
    // of finish_forward (attention.rs:243-253) fused.
    qkv_.wait_for_query_key(rt);
    const Matrix& q = projected.query;
    const Matrix& k = projected.key;
    require(q.cols() == k.cols(), "query/key widths");
    const size_t chunk = score_chunk_rows(q.rows(), k.rows(), max_score_bytes_);
    if (chunk < q.rows()) {
        qkv_.wait_for_value(rt);
        const Matrix& v = projected.value;
        require(v.rows() == k.rows(), "value rows == key rows");
        require(residual.rows() == q.rows() && residual.cols() == v.cols(), "residual shape");
        Matrix out = rt.new_uninit_matrix(q.rows(), v.cols());
        chunked_forward(q, k, v, residual, mask, chunk, out, rt, row_sumsq);
        return out;
    }
    Matrix scores = rt.new_uninit_matrix(q.rows(), k.rows());
    forge_gemm_epilogue ep = plain_epilogue();
    ep.alpha = score_scale(q.cols());
    rt.gemm_ex(nullptr, false, true, q, k, scores.slice(), q.rows(), k.rows(), q.cols(), ep);
    if (mask) scores.causal_mask(rt);
    scores.softmax_rows(rt);
    qkv_.wait_for_value(rt);
    const Matrix& v = projected.value;
    require(v.rows() == k.rows(), "value rows == key rows");
    require(residual.rows() == q.rows() && residual.cols() == v.cols(), "residual shape");
    Matrix out = rt.new_uninit_matrix(q.rows(), v.cols());
    forge_gemm_epilogue ep2 = plain_epilogue();
    ep2.residual = residual.slice();
    if (row_sumsq) ep2.row_sumsq_out = row_sumsq->slice();
    rt.gemm_ex(nullptr, false, false, scores, v, out.slice(), q.rows(), v.cols(), v.rows(), ep2);
    return out;
}

Matrix Attention::forward_pre_norm(const Matrix& query_input, const Matrix& key_value_input,
                                   bool mask, Matrix& row_sumsq, CudaRuntime& rt) {
    // attention.rs:221-241 without the norm: X + A, and the rows' sums of
    // squares from the attention-value product's epilogue.
    const size_t parts = (qkv_.value().weights().cols() + 31) / 32;
    require(row_sumsq.rows() == query_input.rows() && row_sumsq.cols() == parts,
            "row_sumsq shape");
    return attention_value(qkv_.project(query_input, key_value_input, rt), query_input, mask, rt,
                           &row_sumsq);
}

Matrix Attention::forward(const Matrix& query_input, const Matrix& key_value_input,
                          CudaRuntime& rt) {
    // attention.rs:221-230.
    Matrix out = attention_value(qkv_.project(query_input, key_value_input, rt), query_input,
                                 false, rt);
    normalize(out, rt);
    return out;
}

Matrix Attention::forward_mask(const Matrix& query_input, const Matrix& key_value_input,
                               CudaRuntime& rt) {
    // attention.rs:232-241.
    Matrix out = attention_value(qkv_.project(query_input, key_value_input, rt), query_input,
                                 true, rt);
    normalize(out, rt);
    return out;
}

Matrix Attention::forward_self_training(Matrix input, CudaRuntime& rt) {
    // attention.rs:258-281: keeps input, Q, K, V, P and the pre-norm sum.
    QkvProjection::Projected p = qkv_.project(input, input, rt);
    qkv_.wait_for_query_key(rt);
    const size_t chunk = score_chunk_rows(p.query.rows(), p.key.rows(), max_score_bytes_);
    if (chunk < p.query.rows()) {
        // P is not cached: backward recomputes it chunk by chunk.
        qkv_.wait_for_value(rt);
        Matrix pre_norm = rt.new_uninit_matrix(p.query.rows(), p.value.cols());
        chunked_forward(p.query, p.key, p.value, input, false, chunk, pre_norm, rt);
        Matrix output = rt.new_uninit_matrix(pre_norm.rows(), pre_norm.cols());
        norm_.forward_into(pre_norm, output, rt);
        cache_ = Cache{std::move(input), std::move(p.query), std::move(p.key), std::move(p.value),
                       Matrix(), std::move(pre_norm)};
        return output;
    }
    Matrix probabilities = rt.new_uninit_matrix(p.query.rows(), p.key.rows());
    forge_gemm_epilogue ep = plain_epilogue();
    ep.alpha = score_scale(p.query.cols());
    rt.gemm_ex(nullptr, false, true, p.query, p.key, probabilities.slice(), p.query.rows(),
               p.key.rows(), p.query.cols(), ep);
    probabilities.softmax_rows(rt);
    qkv_.wait_for_value(rt);
    Matrix pre_norm = rt.new_uninit_matrix(p.query.rows(), p.value.cols());
    forge_gemm_epilogue ep2 = plain_epilogue();
    ep2.residual = input.slice();
    rt.gemm_ex(nullptr, false, false, probabilities, p.value, pre_norm.slice(), p.query.rows(),
               p.value.cols(), p.value.rows(), ep2);
    // The pre-norm matrix is cached for backward, so the norm writes a new
    // matrix instead of cloning and normalising in place.
    Matrix output = rt.new_uninit_matrix(pre_norm.rows(), pre_norm.cols());
    norm_.forward_into(pre_norm, output, rt);
    cache_ = Cache{std::move(input), std::move(p.query), std::move(p.key), std::move(p.value),
                   std::move(probabilities), std::move(pre_norm)};
    return output;
}

Matrix Attention::backward_self(const Matrix& output_gradient, float learning_rate,
                                CudaRuntime& rt, TransformerGrads* grads,
                                Matrix* input_gradient, Matrix* position) {
    // attention.rs:283-321 with the QKV part of attention.rs:104-144.
    require(cache_.has_value(), "attention forward must run before backward");
    Cache& c = *cache_;
    const size_t S = c.query.rows(), Sk = c.key.rows(), H = c.value.cols();
    if (grads && grads->weights.size() < 3) {
        grads->weights.resize(3);
        grads->biases.resize(3);
    }
    const size_t D = c.query.cols();
    const float scale = score_scale(D);
    // The softmax backward dS = P * (dP - D) * scale (row.rs:216-236) needs
    // each row's D_r = sum_j P_rj dP_rj over the whole [S, Sk] row.  With
    // dP = R V^T that is sum_c R_rc (P V)_rc, and P V = pre_norm - input (the
    // forward's A V product took the input as its residual): the norm
    // backward that forms R also writes scale * D from the [S, H] operands
    // it streams, and each dP product then forms dS in its epilogue
    // (scale * dP - scale * D, times P) -- no [S, Sk] dP matrix and no
    // softmax backward pass.
    const bool fold_ds = S > 0 && Sk > 0;
    std::optional<Vector> row_term;
    if (fold_ds) row_term = Vector(rt.get_uninit_buffer(S));
    Matrix residual_gradient = norm_backward_step(
        norm_, c.pre_norm, output_gradient, learning_rate, rt, grads != nullptr,
        grads ? &grads->norm1_gamma : nullptr, grads ? &grads->norm1_beta : nullptr,
        fold_ds ? &c.input : nullptr, fold_ds ? &*row_term : nullptr, scale);
    // The dS product: dP rows r0 .. r0 + n - 1 against the P rows `p`.
    auto score_gradient_epilogue = [&](forge_slice p, size_t r0, size_t n) {
        forge_gemm_epilogue ep = plain_epilogue();
        ep.alpha = scale;
        ep.row_sub = forge_slice{row_term->buffer().ptr() + r0, n};
        ep.aux_mul = p;
        return ep;
    };

    Matrix query_gradient, key_gradient, value_gradient;
    bool bias_taken[3] = {false, false, false};  // bias gradient and step already taken
    if (c.probabilities.len() == 0 && S > 0 && Sk > 0) {
        // Chunked: per chunk of query rows, P recomputed as in the forward,
        // then dS = P * (R V^T - D) / sqrt(d) (one product), dV += P^T R,
        // dQ = dS K, dK += dS^T Q; dV and dK sum the chunks in order.
        const size_t chunk = score_chunk_rows(S, Sk, max_score_bytes_);
        const size_t cr = std::min(chunk, S);
        Matrix p_c = rt.new_uninit_matrix(cr, Sk), ds_c = rt.new_uninit_matrix(cr, Sk);
        query_gradient = rt.new_uninit_matrix(S, D);
        key_gradient = rt.new_uninit_matrix(Sk, D);
        value_gradient = rt.new_uninit_matrix(Sk, H);
        for (size_t r0 = 0; r0 < S; r0 += chunk) {
            const size_t n = std::min(chunk, S - r0);
            const forge_slice ps{p_c.buffer().ptr(), n * Sk}, dss{ds_c.buffer().ptr(), n * Sk};
            forge_gemm_epilogue ep = plain_epilogue();
            ep.alpha = scale;
            gemm_slices(rt, false, true, rows_of(c.query, r0, n), c.key.slice(), ps, n, Sk, D, ep,
                        "attention scores");
            check(forge_softmax_rows(rt.raw(), nullptr, ps, n, Sk), "softmax_rows");
            gemm_slices(rt, false, true, rows_of(residual_gradient, r0, n), c.value.slice(), dss,
                        n, Sk, H, score_gradient_epilogue(ps, r0, n), "dS");
            forge_gemm_epilogue acc = plain_epilogue();
            if (r0 > 0) acc.residual = value_gradient.slice();
            gemm_slices(rt, true, false, ps, rows_of(residual_gradient, r0, n),
                        value_gradient.slice(), Sk, H, n, acc, "dV");
            gemm_slices(rt, false, false, dss, c.key.slice(), rows_of(query_gradient, r0, n), n,
                        D, Sk, plain_epilogue(), "dQ");
            forge_gemm_epilogue acck = plain_epilogue();
            if (r0 > 0) acck.residual = key_gradient.slice();
            gemm_slices(rt, true, false, dss, rows_of(c.query, r0, n), key_gradient.slice(), Sk,
                        D, n, acck, "dK");
        }
    } else {
        // The projections' G are dQ, dK, dV themselves (identity activation):
        // their bias gradients and SGD steps come from the column sums of
        // the GEMMs that form them.
        auto bias_sums = [&](int i) {
            forge_gemm_epilogue ep = plain_epilogue();
            Linear& lin = i == 0 ? qkv_.query() : i == 1 ? qkv_.key() : qkv_.value();
            if (!lin.bias() || lin.needs_pre_activation()) return ep;
            if (grads) {
                grads->biases[i] = Vector(rt.get_uninit_buffer(lin.bias()->len()));
                ep.col_sums_out = grads->biases[i]->slice();
            }
            ep.col_sums_param = lin.bias()->slice();
            ep.col_sums_lr = learning_rate;
            bias_taken[i] = true;
            return ep;
        };
        // dS = P * (R V^T - D) / sqrt(d) (NT, softmax backward in the
        // epilogue), dV = P^T R (TN).
        Matrix score_gradient = rt.new_uninit_matrix(S, Sk);
        rt.gemm_ex(nullptr, false, true, residual_gradient, c.value, score_gradient.slice(), S, Sk,
                   H, score_gradient_epilogue(c.probabilities.slice(), 0, S));
        value_gradient = rt.new_uninit_matrix(Sk, H);
        rt.gemm_ex(nullptr, true, false, c.probabilities, residual_gradient, value_gradient.slice(),
                   Sk, H, S, bias_sums(2));
        // dQ = dS K (NN), dK = dS^T Q (TN).
        query_gradient = rt.new_uninit_matrix(S, D);
        rt.gemm_ex(nullptr, false, false, score_gradient, c.key, query_gradient.slice(), S, D, Sk,
                   bias_sums(0));
        key_gradient = rt.new_uninit_matrix(Sk, D);
        rt.gemm_ex(nullptr, true, false, score_gradient, c.query, key_gradient.slice(), Sk, D, S,
                   bias_sums(1));
        score_gradient = Matrix();
    }

    // QkvProjection::backward_self: per projection dX accumulates and W, b
    // are updated (dW, db kept when grads are requested).  The input
    // gradient dXp = R + sum_i G_i W_i^T (attention.rs:104-144 plus the
    // residual path) accumulates onto R in place; the last product writes
    // dXp to its target and, with `position`, also takes the position
    // matrix's SGD step from it (pre_out = dXp, C = position updated).
    if (input_gradient)
        require(input_gradient->rows() == residual_gradient.rows() &&
                    input_gradient->cols() == residual_gradient.cols(),
                "input gradient shape");
    if (position)
        require(position->rows() == residual_gradient.rows() &&
                    position->cols() == residual_gradient.cols(),
                "position gradient shape");
    Matrix owned_result;
    Matrix* target = input_gradient;
    if (!target) {
        owned_result = rt.new_uninit_matrix(residual_gradient.rows(), residual_gradient.cols());
        target = &owned_result;
    }
    // The epilogue of the product that completes dXp (residual R, and with
    // `position` the store of dXp and the position step), and its output.
    auto final_epilogue = [&](forge_slice* out) {
        forge_gemm_epilogue ep = plain_epilogue();
        ep.residual = residual_gradient.slice();
        *out = target->slice();
        if (position) {
            ep.pre_out = target->slice();
            ep.update = 1;
            ep.update_scale = learning_rate;
            *out = position->slice();
        }
        return ep;
    };
    auto accumulate_input_gradient = [&](Linear& lin, const Matrix& g, bool last) {
        if (!last) {
            lin.input_gradient_accumulate(g, residual_gradient, rt, nullptr);
            return;
        }
        require(g.cols() == lin.weights().cols(), "gradient.cols() == weights.cols()");
        forge_slice out;
        const forge_gemm_epilogue ep = final_epilogue(&out);
        rt.gemm_ex(nullptr, false, true, g, lin.weights(), out, g.rows(), lin.weights().rows(),
                   lin.weights().cols(), ep);
    };
    Linear* linears[3] = {&qkv_.query(), &qkv_.key(), &qkv_.value()};
    const Matrix* projected[3] = {&query_gradient, &key_gradient, &value_gradient};
    // With identity projections of one weight shape whose biases (if any)
    // took their step in the epilogues above, dXp = R + sum_i G_i W_i^T is
    // one product over three K segments (one read and one write of R's size
    // instead of three of each), and the three weight updates are one
    // batched launch after it.  Each input gradient reads only its own W, so
    // the order of updates and input gradients does not change a result.
    bool batch = true;
    for (int i = 0; i < 3; i++)
        batch = batch && !linears[i]->needs_pre_activation() &&
                (!linears[i]->bias() || bias_taken[i]) &&
                linears[i]->weights().rows() == linears[0]->weights().rows() &&
                linears[i]->weights().cols() == linears[0]->weights().cols();
    if (batch) {
        forge_slice gs[3], ws[3];
        for (int i = 0; i < 3; i++) {
            require(projected[i]->cols() == linears[i]->weights().cols(),
                    "gradient.cols() == weights.cols()");
            gs[i] = projected[i]->slice();
            ws[i] = linears[i]->weights().slice();
        }
        forge_slice out;
        const forge_gemm_epilogue ep = final_epilogue(&out);
        check(forge_gemm_sum_f32(rt.raw(), nullptr, 0, 1, 3, gs, ws, out, projected[0]->rows(),
                                 linears[0]->weights().rows(), linears[0]->weights().cols(),
                                 &ep),
              "qkv input gradients");
        forge_gemm_problem probs[3];
        for (int i = 0; i < 3; i++) {
            Linear& lin = *linears[i];
            Matrix* wg = nullptr;
            if (grads) {
                grads->weights[i] =
                    rt.new_uninit_matrix(lin.weights().rows(), lin.weights().cols());
                wg = &grads->weights[i];
            }
            probs[i] = lin.learn_problem(c.input, *projected[i], learning_rate, wg);
        }
        check(forge_gemm_batch_f32(rt.raw(), nullptr, 1, 0, linears[0]->weights().rows(),
                                   linears[0]->weights().cols(), c.input.rows(), 3, probs),
              "qkv weight updates");
    }
    for (int i = 0; i < 3 && !batch; i++) {
        Linear& lin = *linears[i];
        std::optional<Matrix> g_owned;
        std::optional<Vector> db;
        if (bias_taken[i] && grads) db = std::move(grads->biases[i]);
        const Matrix* g = projected[i];
        if (lin.needs_pre_activation()) {
            Matrix pre = lin.affine(c.input, nullptr, rt, nullptr);
            auto gb = lin.backward(&pre, *projected[i], rt, nullptr);
            g_owned = std::move(gb.first);
            db = std::move(gb.second);
            g = &*g_owned;
        }
        const bool defer_bias = lin.bias() && !db && !bias_taken[i];
        accumulate_input_gradient(lin, *g, i == 2);
        Matrix* wg = nullptr;
        if (grads) {
            grads->weights[i] = rt.new_uninit_matrix(lin.weights().rows(), lin.weights().cols());
            wg = &grads->weights[i];
        }
        if (defer_bias)
            lin.learn_from_gradient(c.input, *g, learning_rate, wg, grads ? &db : nullptr, rt,
                                    nullptr);
        else
            lin.learn_keep(c.input, *g, db ? &*db : nullptr, learning_rate, wg, rt, nullptr,
                           /*bias_step=*/!bias_taken[i]);
        if (grads) grads->biases[i] = std::move(db);
    }
    return owned_result;
}

// ============================================= transformer metadata / data

// inference.rs:52-73 and encoder.rs:90-112: Q, K, V, the position matrix,
// the feed-forward layers and the output projection, then (the gamma/beta
// extension) each norm's gamma and beta that exist, first norm first.
static TransformerMetadata transformer_meta_data(const Attention& attention,
                                                 const Matrix& position, const MlpExecutor& fcs,
                                                 const Linear& output, const Normalization& norm2,
                                                 MetadataCursor& cursor) {
    TransformerMetadata m;
    m.normalization = attention.norm_type();
    m.query = attention.qkv().query().get_meta_data(cursor);
    m.key = attention.qkv().key().get_meta_data(cursor);
    m.value = attention.qkv().value().get_meta_data(cursor);
    m.position = cursor.matrix(position.rows(), position.cols());
    m.feed_forward = fcs.get_meta_data(cursor);
    m.output = output.get_meta_data(cursor);
    const Normalization& norm1 = attention.normalization();
    if (norm1.gamma) m.norm1_gamma = cursor.vector(norm1.gamma->len());
    if (norm1.beta) m.norm1_beta = cursor.vector(norm1.beta->len());
    if (norm2.gamma) m.norm2_gamma = cursor.vector(norm2.gamma->len());
    if (norm2.beta) m.norm2_beta = cursor.vector(norm2.beta->len());
    return m;
}

static std::vector<HostData> transformer_data(const Attention& attention, const Matrix& position,
                                              const MlpExecutor& fcs, const Linear& output,
                                              const Normalization& norm2, CudaRuntime& rt) {
    std::vector<HostData> data;
    auto append = [&data](std::vector<HostData> more) {
        for (HostData& d : more) data.push_back(std::move(d));
    };
    append(attention.qkv().query().get_data(rt));
    append(attention.qkv().key().get_data(rt));
    append(attention.qkv().value().get_data(rt));
    data.emplace_back(position.to_host(rt));
    append(fcs.get_data(rt));
    append(output.get_data(rt));
    const Normalization& norm1 = attention.normalization();
    for (const Normalization* n : {&norm1, &norm2}) {
        if (n->gamma) data.emplace_back(n->gamma->to_host(rt));
        if (n->beta) data.emplace_back(n->beta->to_host(rt));
    }
    return data;
}

// ========================================================= InferenceBlock

static Normalization default_norm(NormType kind) {
    Normalization n;
    n.kind = kind;
    return n;
}

InferenceBlock::InferenceBlock(Linear query, Linear key, Linear value, Matrix position,
                               InferenceMLP fcs, Linear output,
                               std::optional<std::vector<CudaStream>> qkv_streams,
                               NormType norm_type, std::optional<Normalization> norm2)
    : attention_(std::move(query), std::move(key), std::move(value), std::move(qkv_streams),
                 default_norm(norm_type)),
      position_(std::move(position)), fcs_(std::move(fcs)), output_(std::move(output)),
      norm2_(norm2 ? std::move(*norm2) : default_norm(norm_type)) {}

TransformerMetadata InferenceBlock::get_meta_data(MetadataCursor& cursor) const {
    return transformer_meta_data(attention_, position_, fcs_.executor(), output_, norm2_, cursor);
}

std::vector<HostData> InferenceBlock::get_data(CudaRuntime& rt) const {
    return transformer_data(attention_, position_, fcs_.executor(), output_, norm2_, rt);
}

bool InferenceBlock::can_fold_norms() const {
    const Normalization& n1 = attention_.normalization();
    return n1.kind == NormType::Rms && !n1.gamma && !n1.beta && norm2_.kind == NormType::Rms &&
           !norm2_.gamma && !norm2_.beta && !fcs_.executor().res_range();
}

// A Linear's forward (bias, activation) with the row statistics of a
// folded RMSNorm in its epilogue.
static void forward_with_row_stats(const Linear& layer, const Matrix& input, Matrix& out,
                                   const Matrix* residual, const Matrix* parts_in, int row_div,
                                   size_t row_n, float eps, Matrix* sumsq_out, CudaRuntime& rt) {
    forge_gemm_problem pr = layer.forward_problem(input, out);
    forge_gemm_epilogue ep = pr.epilogue;
    if (residual) ep.residual = residual->slice();
    if (parts_in) {
        ep.row_parts_in = parts_in->slice();
        ep.row_parts = parts_in->cols();
        ep.row_n = row_n;
        ep.row_eps = eps;
        ep.row_div = row_div;
    }
    if (sumsq_out) ep.row_sumsq_out = sumsq_out->slice();
    check(forge_gemm_ex_f32(rt.raw(), nullptr, 0, 0, pr.A, pr.B, pr.C, input.rows(),
                            out.cols(), input.cols(), &ep),
          "folded-norm linear");
}

Matrix InferenceBlock::forward_folded(const Matrix& input, bool mask, CudaRuntime& rt,
                                      Matrix* target) {
    // inference.rs:76-108 with both RMSNorms folded: with h1 = pre1 / d1 and
    // h2 = pre2 / d2 (d the rows' RMS, norm.rs:50-69),
    //   pre1 = X + A                        (rows' sums of squares kept)
    //   F    = act((pre1 W1) / d1 + b1) ...  (first FFN layer)
    //   pre2 = F Wn + bn + pre1 / d1        (last FFN layer, sums kept)
    //   out  = (pre2 Wo) / d2 + bo.
    Matrix positioned = rt.matrix_add(input, position_);
    const size_t S = positioned.rows();
    const size_t H = attention_.qkv().value().weights().cols();
    Matrix sq1 = rt.new_uninit_matrix(S, (H + 31) / 32);
    Matrix pre1 = attention_.forward_pre_norm(positioned, positioned, mask, sq1, rt);
    positioned = Matrix();
    std::vector<Linear>& layers = fcs_.executor().layers();
    const size_t L = layers.size();
    const float eps1 = attention_.normalization().eps, eps2 = norm2_.eps;
    Matrix x;  // the current layer's input (pre1 for the first layer)
    Matrix sq2;
    for (size_t i = 0; i < L; i++) {
        const Matrix& in = i == 0 ? pre1 : x;
        Matrix out = rt.new_uninit_matrix(in.rows(), layers[i].weights().cols());
        const bool first = i == 0, last = i + 1 == L;
        int div = (first ? 1 : 0) | (last ? 2 : 0);
        if (last) sq2 = rt.new_uninit_matrix(S, (out.cols() + 31) / 32);
        forward_with_row_stats(layers[i], in, out, last ? &pre1 : nullptr, div ? &sq1 : nullptr,
                               div, H, eps1, last ? &sq2 : nullptr, rt);
        x = std::move(out);
    }
    pre1 = Matrix();
    sq1 = Matrix();
    Matrix result;
    Matrix* dst = target;
    if (!dst) {
        result = rt.new_uninit_matrix(S, output_.weights().cols());
        dst = &result;
    }
    forward_with_row_stats(output_, x, *dst, nullptr, &sq2, 1, x.cols(), eps2, nullptr, rt);
    return result;
}

Matrix InferenceBlock::forward(const Matrix& input, CudaRuntime& rt) {
    // inference.rs:76-80.
    if (fold_norms_ && can_fold_norms()) return forward_folded(input, false, rt, nullptr);
    Matrix positioned = rt.matrix_add(input, position_);
    Matrix x = attention_.forward(positioned, positioned, rt);
    return finish_forward(std::move(positioned), std::move(x), rt, nullptr);
}

Matrix InferenceBlock::forward_mask(const Matrix& input, CudaRuntime& rt) {
    // inference.rs:82-88.
    if (fold_norms_ && can_fold_norms()) return forward_folded(input, true, rt, nullptr);
    Matrix positioned = rt.matrix_add(input, position_);
    Matrix x = attention_.forward_mask(positioned, positioned, rt);
    return finish_forward(std::move(positioned), std::move(x), rt, nullptr);
}

void InferenceBlock::forward_into(const Matrix& input, Matrix& output, CudaRuntime& rt,
                                  bool mask) {
    if (fold_norms_ && can_fold_norms()) {
        require(output.rows() == input.rows() && output.cols() == output_.weights().cols(),
                "output shape");
        (void)forward_folded(input, mask, rt, &output);
        return;
    }
    Matrix positioned = rt.matrix_add(input, position_);
    Matrix x = mask ? attention_.forward_mask(positioned, positioned, rt)
                    : attention_.forward(positioned, positioned, rt);
    finish_forward(std::move(positioned), std::move(x), rt, &output);
}

Matrix InferenceBlock::finish_forward(Matrix positioned, Matrix x, CudaRuntime& rt,
                                      Matrix* target) {
    // inference.rs:90-108: norm(x + ffn(x)) then the output projection; the
    // x + ffn add is fused into the last FFN layer's epilogue.  With a
    // target, the projection writes there and an empty Matrix is returned.
    positioned = Matrix();
    Matrix out = fcs_.executor().forward_plus(x, &x, rt);
    x = Matrix();
    norm2_.forward(out, rt);
    if (target) {
        output_.forward_into(out, nullptr, *target, rt, nullptr);
        return Matrix();
    }
    return output_.forward(out, nullptr, rt, nullptr);
}

namespace encoder {

InferenceTransformer::InferenceTransformer(Linear q, Linear k, Linear v, Matrix position,
                                           InferenceMLP fcs, Linear output,
                                           std::optional<std::vector<CudaStream>> qkv_streams,
                                           NormType norm_type,
                                           std::optional<Normalization> norm1,
                                           std::optional<Normalization> norm2)
    : block_(std::move(q), std::move(k), std::move(v), std::move(position), std::move(fcs),
             std::move(output), std::move(qkv_streams), norm_type, std::move(norm2)) {
    if (norm1) block_.attention().normalization() = std::move(*norm1);
}

TrainingTransformer::TrainingTransformer(Linear q, Linear k, Linear v, Matrix position,
                                         TrainingMlp fcs, Linear output, NormType norm_type,
                                         std::optional<Normalization> norm1,
                                         std::optional<Normalization> norm2)
    : attention_(std::move(q), std::move(k), std::move(v), std::nullopt,
                 norm1 ? std::move(*norm1) : default_norm(norm_type)),
      position_(std::move(position)), fcs_(std::move(fcs)), output_(std::move(output)),
      norm2_(norm2 ? std::move(*norm2) : default_norm(norm_type)) {}

TransformerMetadata TrainingTransformer::get_meta_data(MetadataCursor& cursor) const {
    return transformer_meta_data(attention_, position_, fcs_.executor(), output_, norm2_, cursor);
}

std::vector<HostData> TrainingTransformer::get_data(CudaRuntime& rt) const {
    return transformer_data(attention_, position_, fcs_.executor(), output_, norm2_, rt);
}

Matrix TrainingTransformer::forward(const Matrix& input, CudaRuntime& rt) {
    Matrix output = rt.new_uninit_matrix(input.rows(), output_.weights().cols());
    forward_into(input, output, rt);
    return output;
}

void TrainingTransformer::forward_into(const Matrix& input, Matrix& output, CudaRuntime& rt) {
    // encoder.rs:114-131.
    Matrix positioned = rt.matrix_add(input, position_);
    Matrix first_output = attention_.forward_self_training(std::move(positioned), rt);
    // second_pre_norm = first_output + ffn(first_output), fused.
    Matrix second_pre_norm = fcs_.forward_plus(std::move(first_output), true, rt);
    Matrix encoded = rt.new_uninit_matrix(second_pre_norm.rows(), second_pre_norm.cols());
    norm2_.forward_into(second_pre_norm, encoded, rt);
    output_.forward_into(encoded, nullptr, output, rt, nullptr);
    cache_ = Cache{std::move(second_pre_norm), std::move(encoded)};
}

Matrix TrainingTransformer::backward(const Matrix& output_gradient, float learning_rate,
                                     CudaRuntime& rt) {
    return backward_impl(output_gradient, learning_rate, rt, nullptr);
}

Matrix TrainingTransformer::backward_grads(const Matrix& output_gradient, float learning_rate,
                                           CudaRuntime& rt, TransformerGrads& grads) {
    return backward_impl(output_gradient, learning_rate, rt, &grads);
}

void TrainingTransformer::backward_into(const Matrix& output_gradient, float learning_rate,
                                        CudaRuntime& rt, Matrix& input_gradient,
                                        TransformerGrads* grads) {
    (void)backward_impl(output_gradient, learning_rate, rt, grads, &input_gradient);
}

Matrix TrainingTransformer::backward_impl(const Matrix& output_gradient, float learning_rate,
                                          CudaRuntime& rt, TransformerGrads* grads,
                                          Matrix* input_gradient) {
    // encoder.rs:133-186.
    require(cache_.has_value(), "forward must run before backward");
    Cache& c = *cache_;
    const size_t n_ffn = fcs_.executor().len();
    if (grads) {
        grads->weights.clear();
        grads->biases.clear();
        grads->weights.resize(3 + n_ffn + 1);
        grads->biases.resize(3 + n_ffn + 1);
    }

    // Output projection.
    std::optional<Matrix> g_owned;
    std::optional<Vector> db_o;
    const Matrix* g_o = &output_gradient;
    if (output_.needs_pre_activation()) {
        Matrix pre = output_.affine(c.encoded, nullptr, rt, nullptr);
        auto gb = output_.backward(&pre, output_gradient, rt, nullptr);
        g_owned = std::move(gb.first);
        db_o = std::move(gb.second);
        g_o = &*g_owned;
    }
    const bool defer_bias = output_.bias() && !db_o;
    Matrix encoded_gradient = output_.input_gradient(*g_o, rt, nullptr);
    Matrix* wg_o = nullptr;
    if (grads) {
        grads->weights[3 + n_ffn] =
            rt.new_uninit_matrix(output_.weights().rows(), output_.weights().cols());
        wg_o = &grads->weights[3 + n_ffn];
    }
    if (defer_bias)
        output_.learn_from_gradient(c.encoded, *g_o, learning_rate, wg_o, grads ? &db_o : nullptr,
                                    rt, nullptr);
    else
        output_.learn_keep(c.encoded, *g_o, db_o ? &*db_o : nullptr, learning_rate, wg_o, rt,
                           nullptr);
    if (grads) grads->biases[3 + n_ffn] = std::move(db_o);

    // Second norm (its gamma/beta, when present, take the SGD step too).
    Matrix second_gradient = norm_backward_step(
        norm2_, c.second_pre_norm, encoded_gradient, learning_rate, rt, grads != nullptr,
        grads ? &grads->norm2_gamma : nullptr, grads ? &grads->norm2_beta : nullptr);
    encoded_gradient = Matrix();

    // FFN; the residual gradient (second_gradient + ffn input gradient) is
    // fused into its first layer's input-gradient GEMM.
    std::vector<Matrix> ffn_w;
    std::vector<std::optional<Vector>> ffn_b;
    Matrix first_output_gradient =
        fcs_.backward_grads(second_gradient, learning_rate, rt, grads ? &ffn_w : nullptr,
                            grads ? &ffn_b : nullptr, &second_gradient);
    if (grads) {
        for (size_t i = 0; i < n_ffn; i++) {
            grads->weights[3 + i] = std::move(ffn_w[i]);
            grads->biases[3 + i] = std::move(ffn_b[i]);
        }
    }
    second_gradient = Matrix();

    // Attention (fills grads->weights[0..3) and the first norm).
    // Position matrix: P -= lr * dXp (encoder.rs:180-184: clone, scale,
    // subtract, the same two roundings) in the epilogue of the product that
    // completes dXp.  dXp is not scaled in place, so it is returned as the
    // input gradient without the reference's clone.
    Matrix positioned_owned = attention_.backward_self(first_output_gradient, learning_rate, rt,
                                                       grads, input_gradient, &position_);
    Matrix& positioned_gradient = input_gradient ? *input_gradient : positioned_owned;
    if (grads) grads->position = rt.clone_matrix(positioned_gradient);
    return positioned_owned;
}

}  // namespace encoder
}  // namespace oxforge
