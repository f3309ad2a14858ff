/*
 * oxforge_net.h -- C entry points to the executors of oxforge_net.hpp.
 *
 * The reference calls its executors from Rust (src/net/linear.rs, mlp.rs,
 * transformer/encoder.rs, decoder.rs); these entry points expose the same
 * objects to any FFI caller (the Python tests and the benchmark use them).
 * A model owns copies of its parameters in device memory; inputs and
 * outputs are caller device slices (include/oxforge.h).  Errors are status
 * codes; shape violations (the reference's assert! panics) are
 * FORGE_EINVAL with a message in forge_last_error().
 */
#ifndef OXFORGE_NET_H
#define OXFORGE_NET_H

#include "oxforge.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct forge_net_model forge_net_model;

forge_status forge_net_model_destroy(forge_net_model *model);

/* ---------------------------------------------------------------- Linear */

/* Linear::new(weights [in,out], bias [out] or {NULL,0}, activation)
 * (linear.rs:88-95). */
forge_status forge_net_linear_create(forge_runtime *rt, forge_slice weights,
                                     size_t in, size_t out, forge_slice bias,
                                     int activation, forge_net_model **out_model);
/* Linear::forward (linear.rs:116-132): Y = act(X W + b + R); pre_out
 * ({NULL,0} to skip) receives X W + b + R. */
forge_status forge_net_linear_forward(forge_net_model *m, forge_slice x,
                                      size_t rows, forge_slice residual,
                                      forge_slice y, forge_slice pre_out);
/* Linear::backward (linear.rs:232-306): G = dY * act'(pre), db = colsum G
 * (db_out {NULL,0} to skip; required by the reference when biased). */
forge_status forge_net_linear_backward(forge_net_model *m, forge_slice pre,
                                       forge_slice dy, size_t rows,
                                       forge_slice g_out, forge_slice db_out);
/* Linear::input_gradient (linear.rs:417-444): dX = G W^T. */
forge_status forge_net_linear_input_gradient(forge_net_model *m, forge_slice g,
                                             size_t rows, forge_slice dx);
/* Linear::learn (linear.rs:350-415): W -= lr X^T G; b -= lr db. */
forge_status forge_net_linear_learn(forge_net_model *m, forge_slice x,
                                    forge_slice g, forge_slice db, size_t rows,
                                    float lr);
/* Linear::loss_rows (linear.rs:312-348): per-row mean of 0.5 (o - t)^2. */
forge_status forge_net_linear_loss_rows(forge_runtime *rt, forge_slice output,
                                        forge_slice target, size_t rows,
                                        size_t cols, forge_slice loss);
/* Device view of the current weights (which = 0) or bias (which = 1). */
forge_status forge_net_linear_param(forge_net_model *m, int which,
                                    forge_slice *out);

/* ------------------------------------------------------------------- MLP */

/* InferenceMLP / TrainingMlp (mlp.rs:171-269): n_layers Linear layers with
 * dims[i] -> dims[i+1], activations[i], weights[i], biases[i] ({NULL,0} for
 * none); residual range [res_start, res_end) or res_start = -1 for none. */
forge_status forge_net_mlp_create(forge_runtime *rt, size_t n_layers,
                                  const size_t *dims, const int *activations,
                                  const forge_slice *weights,
                                  const forge_slice *biases, long res_start,
                                  long res_end, int training,
                                  forge_net_model **out_model);
forge_status forge_net_mlp_forward(forge_net_model *m, forge_slice x,
                                   size_t rows, forge_slice y);
/* TrainingMlp::backward (mlp.rs:256-264): SGD on every layer; dx receives
 * the input gradient ({NULL,0} to skip). */
forge_status forge_net_mlp_backward(forge_net_model *m, forge_slice dy,
                                    size_t rows, float lr, forge_slice dx);
forge_status forge_net_mlp_param(forge_net_model *m, size_t layer, int which,
                                 forge_slice *out);

/* ----------------------------------------------------------- transformer */

/* Parameter slots of the single-head Post-Norm block.  Biases and the norm
 * gamma/beta are optional ({NULL,0} = absent, the reference's parameterless
 * norm).  W1/B1 is the hidden -> ffn layer, W2/B2 ffn -> hidden. */
enum forge_transformer_param {
    FORGE_TP_WQ = 0, FORGE_TP_BQ, FORGE_TP_WK, FORGE_TP_BK, FORGE_TP_WV,
    FORGE_TP_BV, FORGE_TP_POS, FORGE_TP_W1, FORGE_TP_B1, FORGE_TP_W2,
    FORGE_TP_B2, FORGE_TP_WO, FORGE_TP_BO, FORGE_TP_G1, FORGE_TP_BE1,
    FORGE_TP_G2, FORGE_TP_BE2, FORGE_TP_COUNT
};

enum forge_transformer_kind {
    FORGE_TK_ENCODER_INFERENCE = 0, /* encoder::InferenceTransformer */
    FORGE_TK_ENCODER_TRAINING = 1,  /* encoder::TrainingTransformer  */
    FORGE_TK_DECODER_INFERENCE = 2  /* decoder::InferenceTransformer */
};

typedef struct forge_transformer_desc {
    size_t seq, hidden, ffn, out;
    int norm_type;      /* 0 = NormType::Rms, 1 = NormType::Layer         */
    int kind;           /* forge_transformer_kind                        */
    int qkv_streams;    /* inference kinds: 1 = Q/K/V each on one of three
                         * forked streams, joined before the scores and
                         * before A.V (attention.rs:65-102); 0 = one batched
                         * GEMM launch on the primary stream.  Results are
                         * bit-identical.  The training kind always batches. */
    int ffn_activation; /* forge_activation of W1 (W2 and WO: identity)   */
} forge_transformer_desc;

forge_status forge_net_transformer_create(forge_runtime *rt,
                                          const forge_transformer_desc *desc,
                                          const forge_slice *params,
                                          forge_net_model **out_model);
/* forward (encoder.rs:53-55, 114-131; decoder.rs:50-52): input [seq,hidden]
 * -> output [seq,out]. */
forge_status forge_net_transformer_forward(forge_net_model *m,
                                           forge_slice input,
                                           forge_slice output);
/* TrainingTransformer::backward (encoder.rs:133-186): gradients, then SGD
 * with lr.  dx ({NULL,0} to skip) receives the input gradient; grads (NULL
 * to skip, or FORGE_TP_COUNT slices with {NULL,0} to skip one) receive the
 * gradient of each parameter before its update. */
forge_status forge_net_transformer_backward(forge_net_model *m, forge_slice dy,
                                            float lr, forge_slice dx,
                                            const forge_slice *grads);
/* Device view of a current parameter ({NULL,0} if absent). */
forge_status forge_net_transformer_param(forge_net_model *m, int slot,
                                         forge_slice *out);
/* Attention::set_max_score_bytes: the largest [seq, seq] score matrix held
 * at once (default 1 GiB); above it attention runs in chunks of query rows
 * and the training step recomputes each chunk's probabilities in backward.
 * No counterpart in the reference, which always forms the whole matrix. */
forge_status forge_net_transformer_set_score_bytes(forge_net_model *m, size_t bytes);
/* InferenceBlock::set_fold_norms for the inference kinds: on (the default)
 * folds the two parameterless RMSNorms (norm.rs:50-69 at inference.rs:90-108,
 * attention.rs:243-253) into the products beside them (the producing
 * product keeps each row's sums of squares, the consuming ones divide by the
 * row's RMS); off runs the reference's launch order.  Applies when both
 * norms are RMSNorm without gamma and the feed-forward network has no inner
 * residual range; otherwise the reference order runs either way.  The
 * training kind, which caches the normalised rows, is FORGE_EINVAL.  No
 * counterpart in the reference. */
forge_status forge_net_transformer_set_fold_norms(forge_net_model *m, int on);

/* ------------------------------------------------------------ checkpoint */

/* Checkpoint format version 1 (include/oxforge_checkpoint.hpp): <path>.toml
 * metadata plus <path>.bin of little-endian f32 parameters.  A path without
 * an extension gets ".toml"; another extension than ".toml" is FORGE_EINVAL
 * (io.rs:20-29).  Invalid files are FORGE_EINVAL, unreadable or unwritable
 * ones FORGE_EIO, each with a message in forge_last_error(). */
enum forge_checkpoint_kind {
    FORGE_CK_LINEAR = 0,               /* load_linear (model.rs:73-76)        */
    FORGE_CK_MLP_INFERENCE = 1,        /* load_inference_mlp (model.rs:108)   */
    FORGE_CK_MLP_TRAINING = 2,         /* load_training_mlp (model.rs:129)    */
    FORGE_CK_ENCODER_INFERENCE = 3,    /* load_transformer (model.rs:150)     */
    FORGE_CK_ENCODER_TRAINING = 4,     /* load_training_transformer (:186)    */
    FORGE_CK_DECODER_INFERENCE = 5     /* extension: same transformer layout  */
};

/* dump_linear / dump_inference_mlp / dump_training_mlp / dump_transformer /
 * dump_training_transformer (model.rs:53-207), chosen by the handle's model. */
forge_status forge_net_checkpoint_save(forge_net_model *m, const char *path);
/* load_* (model.rs:73-207) into a new handle of the given kind.  A
 * transformer loads into a handle only with a two-layer feed-forward network
 * and query/key width equal to the embedding (the parameter slots above);
 * other shapes are FORGE_EINVAL here (the C++ API loads them all). */
forge_status forge_net_checkpoint_load(forge_runtime *rt, const char *path,
                                       int kind, forge_net_model **out_model);
/* Validates metadata and data-file size without a device; copies the model
 * type ("linear", "mlp" or "transformer", NUL-terminated) into model_type
 * (capacity cap >= 12) and the parameter byte count into *data_bytes. */
forge_status forge_checkpoint_inspect(const char *path, char *model_type,
                                      size_t cap, uint64_t *data_bytes);
/* The widths of a handle's model, for callers holding a loaded handle:
 * Linear {in, out}; MLP {in, width of each layer}; transformer {seq, hidden,
 * ffn, out}.  *count receives the number of widths (at most cap written). */
forge_status forge_net_model_dims(forge_net_model *m, size_t *dims, size_t cap,
                                  size_t *count);
/* The descriptor of a transformer handle (as created or as loaded). */
forge_status forge_net_transformer_describe(forge_net_model *m,
                                            forge_transformer_desc *out);

#ifdef __cplusplus
}
#endif
#endif
