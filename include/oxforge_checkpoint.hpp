/*
 * oxforge_checkpoint.hpp -- checkpoint format version 1 for the executors
 * (the reference's net::checkpoint: src/net/checkpoint/io.rs:1-181,
 * model.rs:1-543, src/net/metadata.rs:1-82).
 *
 * Two files per model:
 *   <name>.toml  versioned metadata: format_version = 1, model_type
 *                ("linear" | "mlp" | "transformer"), scalar_type "f32_le",
 *                data_file (a plain file name), data_bytes, and the model's
 *                shapes, activations, loss, residual range and one
 *                [byte_start, byte_end) range per parameter;
 *   <name>.bin   every parameter as contiguous little-endian f32, in the
 *                order of the ranges.
 * A path without an extension gets ".toml"; any other extension is an error
 * (io.rs:20-29).  Loading validates the version, model type, scalar type,
 * that the ranges are contiguous from 0 and end at data_bytes, the data file
 * size, every tensor shape, Linear connectivity, the residual range and the
 * transformer dimensions (model.rs:353-543), then builds the model through
 * its public constructors.  Errors are oxforge::Error (FORGE_EINVAL for bad
 * data, FORGE_EIO for a file that cannot be opened, read or written).
 *
 * Extension: a transformer whose norms carry gamma/beta writes them as
 * optional tables norm1_gamma, norm1_beta, norm2_gamma, norm2_beta after the
 * reference's parameters.  A file without them is exactly the reference's
 * format; one with them is not loadable by the reference (its range check
 * stops at the output projection).  decoder::InferenceTransformer, which the
 * reference does not checkpoint, uses the transformer layout unchanged.
 */
#ifndef OXFORGE_CHECKPOINT_HPP
#define OXFORGE_CHECKPOINT_HPP

#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "oxforge_net.hpp"

namespace oxforge {
namespace checkpoint {

constexpr uint32_t FORMAT_VERSION = 1;  // model.rs:17

// The metadata types of the executors' get_meta_data (oxforge_net.hpp:
// metadata.rs:5-18, linear.rs:79-86, mlp.rs:21-34, inference.rs:12-24).
using oxforge::LinearMetadata;
using oxforge::MatrixMetadata;
using oxforge::MlpMetadata;
using oxforge::ResidualMetadata;
using oxforge::TransformerMetadata;
using oxforge::VectorMetadata;

// model.rs:53-207 entry points.
void dump_linear(Linear& model, const std::string& path, CudaRuntime& rt);
Linear load_linear(const std::string& path, CudaRuntime& rt);
void dump_mlp(MlpExecutor& model, const std::string& path, CudaRuntime& rt);
MlpExecutor load_mlp(const std::string& path, CudaRuntime& rt);
void dump_inference_mlp(InferenceMLP& model, const std::string& path, CudaRuntime& rt);
InferenceMLP load_inference_mlp(const std::string& path, CudaRuntime& rt);
void dump_training_mlp(TrainingMlp& model, const std::string& path, CudaRuntime& rt);
TrainingMlp load_training_mlp(const std::string& path, CudaRuntime& rt);
void dump_transformer(encoder::InferenceTransformer& model, const std::string& path,
                      CudaRuntime& rt);
encoder::InferenceTransformer load_transformer(const std::string& path, CudaRuntime& rt);
void dump_training_transformer(encoder::TrainingTransformer& model, const std::string& path,
                               CudaRuntime& rt);
encoder::TrainingTransformer load_training_transformer(const std::string& path,
                                                       CudaRuntime& rt);
// Extension: the causal-mask block in the same transformer layout.
void dump_decoder_transformer(decoder::InferenceTransformer& model, const std::string& path,
                              CudaRuntime& rt);
decoder::InferenceTransformer load_decoder_transformer(const std::string& path, CudaRuntime& rt);

// Parses and validates a checkpoint's metadata and data-file size without
// touching a device; returns the model type and sets *data_bytes.
std::string inspect(const std::string& path, uint64_t* data_bytes);
// The metadata of a transformer checkpoint (validated), for callers that
// need its dimensions before loading.
TransformerMetadata read_transformer_metadata(const std::string& path);

}  // namespace checkpoint
}  // namespace oxforge

#endif
