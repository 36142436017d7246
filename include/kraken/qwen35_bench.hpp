// kraken/qwen35_bench.hpp -- the reference's hot-path micro-benchmarks over the
// HIP backend, header-only C++17:
//   benchmark_gdn / format_gdn_bench_result mirror benchmark_qwen35_metal_gdn /
//     format_qwen35_gdn_bench_result (qwen35_runtime.cpp:4808-4994);
//   benchmark_attention / format_attention_bench_result mirror
//     benchmark_qwen35_metal_attention / format_qwen35_attention_bench_result
//     (qwen35_runtime.cpp:4997-5236);
//   benchmark_matmul / format_matmul_bench_result mirror
//     benchmark_qwen35_metal_matmul / format_qwen35_matmul_bench_result
//     (qwen35_runtime.cpp:4558-4806): one K-quant tensor of a GGUF file times a
//     tokens x cols input on matmul_q{4,5,6}_k_f32_device;
//   the config and result types mirror Qwen35{Matmul,Gdn,Attention}Bench{Config,Result}
//     (qwen35_runtime.hpp:75-175), with the same defaults.
// Same argument checks and messages, same deterministic modular inputs, same
// loop (warmup, then timed iterations of one graph each: begin, op, commit,
// which waits), same derived rates and the same 16-value weighted checksum of
// the output.  The dispatch string names this backend's kernel for the shape.
#pragma once

#include <algorithm>
#include <chrono>
#include <filesystem>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <sstream>
#include <string>
#include <vector>

#include "kraken/gguf.hpp"
#include "kraken/hip_context.hpp"

namespace kraken {
namespace qwen35 {

struct MatmulBenchConfig {
  std::string model_path;  // a .gguf file, or a directory holding one
  std::string tensor_name;
  std::size_t tokens{1024};
  std::size_t warmup_iterations{2};
  std::size_t timed_iterations{10};
};

struct MatmulBenchResult {
  std::string gguf_path;
  std::string tensor_name;
  std::string type_name;
  std::string dispatch;
  std::uint32_t type{0};
  std::size_t tokens{0};
  std::size_t rows{0};
  std::size_t cols{0};
  std::size_t warmup_iterations{0};
  std::size_t timed_iterations{0};
  std::uint64_t output_values_per_iteration{0};
  double total_seconds{0.0};
  double average_milliseconds{0.0};
  double token_iterations_per_second{0.0};
  double output_megavalues_per_second{0.0};
  double sample_checksum{0.0};
};

struct GdnBenchConfig {
  std::size_t tokens{1024};
  std::size_t key_heads{16};
  std::size_t value_heads{16};
  std::size_t head_dim{128};
  std::size_t warmup_iterations{2};
  std::size_t timed_iterations{10};
};

struct GdnBenchResult {
  std::string dispatch;
  std::size_t tokens{0};
  std::size_t key_heads{0};
  std::size_t value_heads{0};
  std::size_t head_dim{0};
  std::size_t warmup_iterations{0};
  std::size_t timed_iterations{0};
  std::uint64_t state_values{0};
  std::uint64_t output_values_per_iteration{0};
  double total_seconds{0.0};
  double average_milliseconds{0.0};
  double token_iterations_per_second{0.0};
  double output_megavalues_per_second{0.0};
  double sample_checksum{0.0};
};

struct AttentionBenchConfig {
  std::size_t tokens{1024};
  std::size_t start_position{0};
  std::size_t capacity_tokens{0};
  std::size_t heads{8};
  std::size_t kv_heads{2};
  std::size_t head_dim{256};
  std::size_t warmup_iterations{2};
  std::size_t timed_iterations{10};
  bool f16_kv{true};
};

struct AttentionBenchResult {
  std::string dispatch;
  std::size_t tokens{0};
  std::size_t start_position{0};
  std::size_t capacity_tokens{0};
  std::size_t key_count{0};
  std::size_t heads{0};
  std::size_t kv_heads{0};
  std::size_t head_dim{0};
  std::size_t warmup_iterations{0};
  std::size_t timed_iterations{0};
  std::uint64_t cache_values{0};
  std::uint64_t output_values_per_iteration{0};
  double total_seconds{0.0};
  double average_milliseconds{0.0};
  double token_iterations_per_second{0.0};
  double output_megavalues_per_second{0.0};
  double sample_checksum{0.0};
  bool f16_kv{true};
};

namespace bench_detail {

inline bool checked_mul_size(std::size_t a, std::size_t b, std::size_t& out) {
  if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) {
    return false;
  }
  out = a * b;
  return true;
}

// make_qwen35_f32_buffer: a device buffer holding `values` (or `count` zeros).
inline hip::Result<hip::HipBuffer> f32_buffer(const hip::HipContext& context,
                                              const std::vector<float>& values) {
  auto buffer = context.make_buffer(values.size() * sizeof(float));
  if (!buffer.is_ok()) {
    return buffer.status();
  }
  const hip::Status s =
    context.copy_to_buffer(buffer.value(), values.data(), values.size() * sizeof(float));
  if (!s.is_ok()) {
    return s;
  }
  return std::move(buffer.value());
}

// Weighted sum of the first 16 output values (weights 1..16), in double.
inline hip::Result<double> sample_checksum(const hip::HipContext& context,
                                           const hip::HipBuffer& output, std::size_t values) {
  std::vector<float> sample(std::min<std::size_t>(values, 16U), 0.0F);
  const hip::Status s =
    context.copy_from_buffer(output, sample.data(), sample.size() * sizeof(float));
  if (!s.is_ok()) {
    return s;
  }
  double checksum = 0.0;
  for (std::size_t index = 0; index < sample.size(); ++index) {
    checksum += static_cast<double>(sample[index]) * static_cast<double>(index + 1U);
  }
  return checksum;
}

// Warmup, then the timed loop; each iteration is one graph (begin, op, commit).
// Returns the timed seconds.
template <typename Op>
hip::Result<double> timed_graph_loop(const hip::HipContext& context, std::size_t warmup,
                                     std::size_t timed, Op op) {
  auto run_once = [&]() -> hip::Status {
    hip::Status s = context.begin_graph();
    if (!s.is_ok()) {
      return s;
    }
    s = op();
    if (!s.is_ok()) {
      context.abort_graph();
      return s;
    }
    return context.commit_graph();
  };
  for (std::size_t i = 0; i < warmup; ++i) {
    const hip::Status s = run_once();
    if (!s.is_ok()) {
      return s;
    }
  }
  const auto start = std::chrono::steady_clock::now();
  for (std::size_t i = 0; i < timed; ++i) {
    const hip::Status s = run_once();
    if (!s.is_ok()) {
      return s;
    }
  }
  const auto end = std::chrono::steady_clock::now();
  return std::chrono::duration<double>(end - start).count();
}

inline bool env_is(const char* name, const char* value) {
  const char* v = std::getenv(name);
  return v != nullptr && std::strcmp(v, value) == 0;
}

}  // namespace bench_detail

// The GDN kernel this backend runs for the shape (KRAKEN_GDN_PREFILL overrides
// the head_dim-128 multi-token choice).
inline std::string gdn_dispatch_name(std::size_t tokens, std::size_t head_dim) {
  if (head_dim != 128U || bench_detail::env_is("KRAKEN_GDN_PREFILL", "generic")) {
    return "generic_batched_gdn";
  }
  if (tokens >= 64U && !bench_detail::env_is("KRAKEN_GDN_PREFILL", "sequential")) {
    return "chunked_wy";
  }
  return "recurrence_128";
}

// The attention kernel this backend runs: flash256 for head_dim 256, tokens >= 64
// and an F16 cache (KRAKEN_QWEN35_FLASH_ATTENTION=1/0 forces it on/off), else the
// split-KV decode kernel.
inline std::string attention_dispatch_name(std::size_t tokens, std::size_t head_dim,
                                           bool f16_kv) {
  const char* v = std::getenv("KRAKEN_QWEN35_FLASH_ATTENTION");
  const bool on = v != nullptr && (std::strcmp(v, "1") == 0 || std::strcmp(v, "true") == 0 ||
                                   std::strcmp(v, "on") == 0);
  const bool off = v != nullptr && (std::strcmp(v, "0") == 0 || std::strcmp(v, "false") == 0 ||
                                    std::strcmp(v, "off") == 0);
  if (f16_kv && head_dim == 256U && !off && (on || tokens >= 64U)) {
    return "flash256_f16_kv";
  }
  return f16_kv ? "split_kv_decode_f16_kv" : "split_kv_decode_f32";
}

// resolve_gguf_model_path (gguf_reader.cpp:521-546): a .gguf file as given, or
// the first .gguf (by name) in a directory.
inline hip::Result<std::string> resolve_gguf_path(const std::string& path) {
  namespace fs = std::filesystem;
  std::error_code ec;
  const fs::path p(path);
  if (!fs::exists(p, ec)) {
    return hip::Status::unavailable("model path does not exist: " + path);
  }
  if (fs::is_regular_file(p, ec)) {
    if (p.extension() == ".gguf") {
      return path;
    }
    return hip::Status::invalid_argument("model file is not a GGUF file: " + path);
  }
  if (!fs::is_directory(p, ec)) {
    return hip::Status::invalid_argument("model path is not a file or directory: " + path);
  }
  std::vector<std::string> candidates;
  for (const auto& entry : fs::directory_iterator(p, ec)) {
    if (entry.is_regular_file() && entry.path().extension() == ".gguf") {
      candidates.push_back(entry.path().string());
    }
  }
  if (candidates.empty()) {
    return hip::Status::unavailable("no GGUF file found in " + path);
  }
  std::sort(candidates.begin(), candidates.end());
  return candidates.front();
}

// The name of a GGUF tensor type id (ggml's table).
inline std::string ggml_type_name(std::uint32_t type) {
  static const char* const kNames[] = {"F32",  "F16",  "Q4_0", "Q4_1", "", "",
                                       "Q5_0", "Q5_1", "Q8_0", "Q8_1", "Q2_K", "Q3_K",
                                       "Q4_K", "Q5_K", "Q6_K", "Q8_K"};
  if (type < sizeof(kNames) / sizeof(kNames[0]) && kNames[type][0] != '\0') {
    return kNames[type];
  }
  return "type_" + std::to_string(type);
}

// The K-quant projection kernel this backend runs for `tokens` rows of input
// (capi_kquant: the fp32 GEMV up to 3 tokens, the GEMV on fp16-rounded weights
// for 4 to 8, the fp16 MFMA GEMM above 8).
inline std::string kquant_matmul_dispatch_name(std::uint32_t type, std::size_t tokens) {
  if (type != 12U && type != 13U && type != 14U) {
    return "unsupported";
  }
  if (tokens > 8U) {
    return "kquant_gemm_f16_mfma";
  }
  return tokens >= 4U ? "kquant_gemv_f16_weights" : "kquant_gemv_f32";
}

// benchmark_qwen35_metal_matmul (qwen35_runtime.cpp:4558-4782).
inline hip::Result<MatmulBenchResult> benchmark_matmul(const MatmulBenchConfig& config) {
  using hip::Status;
  if (config.model_path.empty()) {
    return Status::invalid_argument("Qwen3.5 matmul bench requires --model");
  }
  if (config.tensor_name.empty()) {
    return Status::invalid_argument("Qwen3.5 matmul bench requires --tensor");
  }
  if (config.tokens == 0) {
    return Status::invalid_argument("Qwen3.5 matmul bench tokens must be positive");
  }
  if (config.timed_iterations == 0) {
    return Status::invalid_argument("Qwen3.5 matmul bench timed iterations must be positive");
  }
  auto path = resolve_gguf_path(config.model_path);
  if (!path.is_ok()) {
    return path.status();
  }
  auto file = gguf::read_file(path.value());
  if (!file.is_ok()) {
    return file.status();
  }
  const gguf::TensorInfo* tensor = gguf::find_tensor(file.value(), config.tensor_name);
  if (tensor == nullptr) {
    return Status::invalid_argument("Qwen3.5 matmul bench tensor not found: " +
                                    config.tensor_name);
  }
  if (tensor->shape.size() != 2U) {
    return Status::invalid_argument("Qwen3.5 matmul bench tensor must be 2D: " + tensor->name);
  }
  if (tensor->type != 12U && tensor->type != 13U && tensor->type != 14U) {
    return Status::invalid_argument(
      "Qwen3.5 matmul bench currently supports only Q4_K/Q5_K/Q6_K tensors: " + tensor->name);
  }
  if (tensor->shape[0] > std::numeric_limits<std::size_t>::max() ||
      tensor->shape[1] > std::numeric_limits<std::size_t>::max()) {
    return Status::invalid_argument(tensor->name + " exceeds size_t");
  }
  const auto cols = static_cast<std::size_t>(tensor->shape[0]);
  const auto rows = static_cast<std::size_t>(tensor->shape[1]);
  if (cols == 0 || rows == 0) {
    return Status::invalid_argument("Qwen3.5 matmul bench tensor shape is empty: " +
                                    tensor->name);
  }
  if (cols % 256U != 0) {
    return Status::invalid_argument("Qwen3.5 matmul bench K-quant cols must be divisible by 256: " +
                                    tensor->name);
  }
  std::size_t input_values = 0;
  std::size_t output_values = 0;
  std::size_t bytes = 0;
  if (!bench_detail::checked_mul_size(config.tokens, cols, input_values) ||
      !bench_detail::checked_mul_size(config.tokens, rows, output_values) ||
      !bench_detail::checked_mul_size(input_values, sizeof(float), bytes) ||
      !bench_detail::checked_mul_size(output_values, sizeof(float), bytes)) {
    return Status::invalid_argument("Qwen3.5 matmul bench value count overflow");
  }
  auto mapped = gguf::MappedData::open(file.value());
  if (!mapped.is_ok()) {
    return mapped.status();
  }
  auto weight_bytes = mapped.value().tensor_bytes(*tensor);
  if (!weight_bytes.is_ok()) {
    return weight_bytes.status();
  }

  auto context = hip::HipContext::create();
  if (!context.is_ok()) {
    return context.status();
  }
  const hip::HipContext& ctx = context.value();
  auto weight = ctx.make_buffer(weight_bytes.value().second);
  if (!weight.is_ok()) {
    return weight.status();
  }
  Status status =
    ctx.copy_to_buffer(weight.value(), weight_bytes.value().first, weight_bytes.value().second);
  if (!status.is_ok()) {
    return status;
  }
  // The reference's input pattern: (index mod 23 - 11) / 32.
  std::vector<float> input(input_values);
  for (std::size_t i = 0; i < input.size(); ++i) {
    input[i] = static_cast<float>(static_cast<int>(i % 23U) - 11) * 0.03125F;
  }
  auto input_buffer = bench_detail::f32_buffer(ctx, input);
  if (!input_buffer.is_ok()) {
    return input_buffer.status();
  }
  auto output = ctx.make_buffer(output_values * sizeof(float));
  if (!output.is_ok()) {
    return output.status();
  }
  status = ctx.zero_buffer(output.value(), output_values * sizeof(float));
  if (!status.is_ok()) {
    return status;
  }
  const std::uint32_t type = tensor->type;
  auto seconds = bench_detail::timed_graph_loop(
    ctx, config.warmup_iterations, config.timed_iterations, [&]() -> Status {
      switch (type) {
        case 12:
          return ctx.matmul_q4_k_f32_device(weight.value(), rows, cols, config.tokens,
                                            input_buffer.value(), output.value());
        case 13:
          return ctx.matmul_q5_k_f32_device(weight.value(), rows, cols, config.tokens,
                                            input_buffer.value(), output.value());
        default:
          return ctx.matmul_q6_k_f32_device(weight.value(), rows, cols, config.tokens,
                                            input_buffer.value(), output.value());
      }
    });
  if (!seconds.is_ok()) {
    return seconds.status();
  }
  auto checksum = bench_detail::sample_checksum(ctx, output.value(), output_values);
  if (!checksum.is_ok()) {
    return checksum.status();
  }
  MatmulBenchResult r;
  r.gguf_path = path.value();
  r.tensor_name = tensor->name;
  r.type_name = ggml_type_name(type);
  r.dispatch = kquant_matmul_dispatch_name(type, config.tokens);
  r.type = type;
  r.tokens = config.tokens;
  r.rows = rows;
  r.cols = cols;
  r.warmup_iterations = config.warmup_iterations;
  r.timed_iterations = config.timed_iterations;
  r.output_values_per_iteration = output_values;
  r.total_seconds = seconds.value();
  const double timed = static_cast<double>(config.timed_iterations);
  r.average_milliseconds = r.total_seconds * 1000.0 / timed;
  r.token_iterations_per_second = static_cast<double>(config.tokens) * timed / r.total_seconds;
  r.output_megavalues_per_second =
    static_cast<double>(output_values) * timed / (r.total_seconds * 1.0e6);
  r.sample_checksum = checksum.value();
  return r;
}

// format_qwen35_matmul_bench_result (qwen35_runtime.cpp:4784-4806); the first
// line names this backend.
inline std::string format_matmul_bench_result(const MatmulBenchResult& r) {
  std::ostringstream o;
  o << "Qwen3.5 HIP matmul bench: ok\n";
  o << "GGUF: " << r.gguf_path << '\n';
  o << "Tensor: " << r.tensor_name << '\n';
  o << "Type: " << r.type_name << " (" << r.type << ")\n";
  o << "Dispatch: " << r.dispatch << '\n';
  o << "Shape: rows=" << r.rows << ", cols=" << r.cols << ", tokens=" << r.tokens << '\n';
  o << "Iterations: warmup=" << r.warmup_iterations << ", timed=" << r.timed_iterations << '\n';
  o << "Output values/iter: " << r.output_values_per_iteration << '\n';
  o << "Total seconds: " << r.total_seconds << '\n';
  o << "Average ms/iter: " << r.average_milliseconds << '\n';
  o << "Token-iterations/s: " << r.token_iterations_per_second << '\n';
  o << "Output Mvalues/s: " << r.output_megavalues_per_second << '\n';
  o << "Sample checksum: " << r.sample_checksum << '\n';
  return o.str();
}

// benchmark_qwen35_metal_gdn (qwen35_runtime.cpp:4808-4975).
inline hip::Result<GdnBenchResult> benchmark_gdn(const GdnBenchConfig& config) {
  using bench_detail::checked_mul_size;
  if (config.tokens == 0 || config.key_heads == 0 || config.value_heads == 0 ||
      config.head_dim == 0) {
    return hip::Status::invalid_argument("Qwen3.5 GDN bench dimensions must be positive");
  }
  if (config.timed_iterations == 0) {
    return hip::Status::invalid_argument("Qwen3.5 GDN bench timed iterations must be positive");
  }
  std::size_t key_dim = 0, value_dim = 0, qk_values = 0, value_values = 0, gate_values = 0,
              state_rows = 0, state_values = 0;
  if (!checked_mul_size(config.key_heads, config.head_dim, key_dim) ||
      !checked_mul_size(config.value_heads, config.head_dim, value_dim) ||
      !checked_mul_size(config.tokens, key_dim, qk_values) ||
      !checked_mul_size(config.tokens, value_dim, value_values) ||
      !checked_mul_size(config.tokens, config.value_heads, gate_values) ||
      !checked_mul_size(config.value_heads, config.head_dim, state_rows) ||
      !checked_mul_size(state_rows, config.head_dim, state_values)) {
    return hip::Status::invalid_argument("Qwen3.5 GDN bench value count overflow");
  }

  auto context_result = hip::HipContext::create();
  if (!context_result.is_ok()) {
    return context_result.status();
  }
  const hip::HipContext& context = context_result.value();

  // qwen35_runtime.cpp:4846-4862.
  std::vector<float> query(qk_values), key(qk_values), value(value_values), gate(gate_values),
    beta(gate_values), state(state_values);
  for (std::size_t i = 0; i < qk_values; ++i) {
    query[i] = 0.001F * static_cast<float>(1U + i % 17U);
    key[i] = 0.0007F * static_cast<float>(1U + i % 19U);
  }
  for (std::size_t i = 0; i < value_values; ++i) {
    value[i] = 0.002F * static_cast<float>(1U + i % 23U);
  }
  for (std::size_t i = 0; i < gate_values; ++i) {
    gate[i] = -0.002F * static_cast<float>(1U + i % 7U);
    beta[i] = 0.25F + 0.01F * static_cast<float>(i % 11U);
  }
  for (std::size_t i = 0; i < state_values; ++i) {
    state[i] = 0.0001F * static_cast<float>(1U + i % 13U);
  }
  auto q = bench_detail::f32_buffer(context, query);
  auto k = bench_detail::f32_buffer(context, key);
  auto v = bench_detail::f32_buffer(context, value);
  auto g = bench_detail::f32_buffer(context, gate);
  auto b = bench_detail::f32_buffer(context, beta);
  auto s = bench_detail::f32_buffer(context, state);
  auto out = context.make_buffer(value_values * sizeof(float));
  for (const hip::Status* st : {&q.status(), &k.status(), &v.status(), &g.status(),
                                &b.status(), &s.status(), &out.status()}) {
    if (!st->is_ok()) {
      return *st;
    }
  }
  hip::Status status = context.zero_buffer(out.value(), value_values * sizeof(float));
  if (!status.is_ok()) {
    return status;
  }
  // The state is updated in place every iteration, as in the reference.
  auto seconds = bench_detail::timed_graph_loop(
    context, config.warmup_iterations, config.timed_iterations, [&]() {
      return context.gated_delta_net_f32_batched_in_place(
        q.value(), k.value(), v.value(), g.value(), b.value(), s.value(), config.tokens,
        config.key_heads, config.value_heads, config.head_dim, out.value());
    });
  if (!seconds.is_ok()) {
    return seconds.status();
  }
  auto checksum = bench_detail::sample_checksum(context, out.value(), value_values);
  if (!checksum.is_ok()) {
    return checksum.status();
  }
  const double total_seconds = seconds.value();
  const auto timed = static_cast<double>(config.timed_iterations);
  GdnBenchResult result;
  result.dispatch = gdn_dispatch_name(config.tokens, config.head_dim);
  result.tokens = config.tokens;
  result.key_heads = config.key_heads;
  result.value_heads = config.value_heads;
  result.head_dim = config.head_dim;
  result.warmup_iterations = config.warmup_iterations;
  result.timed_iterations = config.timed_iterations;
  result.state_values = static_cast<std::uint64_t>(state_values);
  result.output_values_per_iteration = static_cast<std::uint64_t>(value_values);
  result.total_seconds = total_seconds;
  result.average_milliseconds = total_seconds * 1000.0 / timed;
  result.token_iterations_per_second = static_cast<double>(config.tokens) * timed / total_seconds;
  result.output_megavalues_per_second =
    static_cast<double>(value_values) * timed / (total_seconds * 1000000.0);
  result.sample_checksum = checksum.value();
  return result;
}

// format_qwen35_gdn_bench_result (qwen35_runtime.cpp:4977-4994).
inline std::string format_gdn_bench_result(const GdnBenchResult& result) {
  std::ostringstream output;
  output << "Qwen3.5 HIP GDN bench: ok\n";
  output << "Dispatch: " << result.dispatch << '\n';
  output << "Shape: tokens=" << result.tokens << ", key_heads=" << result.key_heads
         << ", value_heads=" << result.value_heads << ", head_dim=" << result.head_dim << '\n';
  output << "Iterations: warmup=" << result.warmup_iterations
         << ", timed=" << result.timed_iterations << '\n';
  output << "State values: " << result.state_values << '\n';
  output << "Output values/iter: " << result.output_values_per_iteration << '\n';
  output << "Total seconds: " << result.total_seconds << '\n';
  output << "Average ms/iter: " << result.average_milliseconds << '\n';
  output << "Token-iterations/s: " << result.token_iterations_per_second << '\n';
  output << "Output Mvalues/s: " << result.output_megavalues_per_second << '\n';
  output << "Sample checksum: " << result.sample_checksum << '\n';
  return output.str();
}

// benchmark_qwen35_metal_attention (qwen35_runtime.cpp:4997-5212).
inline hip::Result<AttentionBenchResult> benchmark_attention(const AttentionBenchConfig& config) {
  using bench_detail::checked_mul_size;
  if (config.tokens == 0 || config.heads == 0 || config.kv_heads == 0 || config.head_dim == 0) {
    return hip::Status::invalid_argument("Qwen3.5 attention bench dimensions must be positive");
  }
  if (config.heads % config.kv_heads != 0) {
    return hip::Status::invalid_argument(
      "Qwen3.5 attention bench heads must be divisible by kv_heads");
  }
  if (config.head_dim > 256U) {
    return hip::Status::invalid_argument("Qwen3.5 attention bench head_dim must be at most 256");
  }
  if (config.timed_iterations == 0) {
    return hip::Status::invalid_argument(
      "Qwen3.5 attention bench timed iterations must be positive");
  }
  if (config.start_position > std::numeric_limits<std::size_t>::max() - config.tokens) {
    return hip::Status::invalid_argument("Qwen3.5 attention bench key count overflow");
  }
  const std::size_t key_count = config.start_position + config.tokens;
  const std::size_t capacity_tokens =
    config.capacity_tokens == 0 ? key_count : config.capacity_tokens;
  if (key_count > capacity_tokens) {
    return hip::Status::invalid_argument("Qwen3.5 attention bench chunk exceeds capacity_tokens");
  }
  std::size_t attn_dim = 0, kv_dim = 0, query_values = 0, cache_values = 0, f16_cache_bytes = 0;
  if (!checked_mul_size(config.heads, config.head_dim, attn_dim) ||
      !checked_mul_size(config.kv_heads, config.head_dim, kv_dim) ||
      !checked_mul_size(config.tokens, attn_dim, query_values) ||
      !checked_mul_size(capacity_tokens, kv_dim, cache_values) ||
      !checked_mul_size(cache_values, sizeof(std::uint16_t), f16_cache_bytes)) {
    return hip::Status::invalid_argument("Qwen3.5 attention bench value count overflow");
  }

  auto context_result = hip::HipContext::create();
  if (!context_result.is_ok()) {
    return context_result.status();
  }
  const hip::HipContext& context = context_result.value();

  // qwen35_runtime.cpp:5050-5062.
  std::vector<float> query(query_values), key_cache(cache_values), value_cache(cache_values);
  for (std::size_t i = 0; i < query.size(); ++i) {
    query[i] = static_cast<float>(static_cast<int>((i * 13U) % 31U) - 15) * 0.015F;
  }
  for (std::size_t i = 0; i < key_cache.size(); ++i) {
    key_cache[i] = static_cast<float>(static_cast<int>((i * 7U) % 29U) - 14) * 0.012F;
    value_cache[i] = static_cast<float>(static_cast<int>((i * 11U) % 37U) - 18) * 0.025F;
  }
  auto q = bench_detail::f32_buffer(context, query);
  if (!q.is_ok()) {
    return q.status();
  }
  auto k32 = bench_detail::f32_buffer(context, key_cache);
  auto v32 = bench_detail::f32_buffer(context, value_cache);
  if (!k32.is_ok()) {
    return k32.status();
  }
  if (!v32.is_ok()) {
    return v32.status();
  }
  hip::HipBuffer kc, vc;
  hip::Status status;
  if (config.f16_kv) {
    // The F16 caches are made on the device from the F32 values (RNE), as the
    // reference does with copy_f32_rows_to_f16.
    auto kh = context.make_buffer(f16_cache_bytes);
    auto vh = context.make_buffer(f16_cache_bytes);
    if (!kh.is_ok()) {
      return kh.status();
    }
    if (!vh.is_ok()) {
      return vh.status();
    }
    status = context.copy_f32_rows_to_f16(k32.value(), kh.value(), capacity_tokens, kv_dim, kv_dim,
                                          0, kv_dim, 0);
    if (!status.is_ok()) {
      return status;
    }
    status = context.copy_f32_rows_to_f16(v32.value(), vh.value(), capacity_tokens, kv_dim, kv_dim,
                                          0, kv_dim, 0);
    if (!status.is_ok()) {
      return status;
    }
    kc = std::move(kh.value());
    vc = std::move(vh.value());
  } else {
    kc = std::move(k32.value());
    vc = std::move(v32.value());
  }
  auto out = context.make_buffer(query_values * sizeof(float));
  if (!out.is_ok()) {
    return out.status();
  }
  status = context.zero_buffer(out.value(), query_values * sizeof(float));
  if (!status.is_ok()) {
    return status;
  }
  auto seconds = bench_detail::timed_graph_loop(
    context, config.warmup_iterations, config.timed_iterations, [&]() {
      return config.f16_kv
               ? context.attention_f32_batched_f16_kv(
                   q.value(), kc, vc, 0, config.start_position, config.tokens, capacity_tokens,
                   config.heads, config.kv_heads, config.head_dim, out.value())
               : context.attention_f32_batched(q.value(), kc, vc, 0, config.start_position,
                                               config.tokens, capacity_tokens, config.heads,
                                               config.kv_heads, config.head_dim, out.value());
    });
  if (!seconds.is_ok()) {
    return seconds.status();
  }
  auto checksum = bench_detail::sample_checksum(context, out.value(), query_values);
  if (!checksum.is_ok()) {
    return checksum.status();
  }
  const double total_seconds = seconds.value();
  const auto timed = static_cast<double>(config.timed_iterations);
  AttentionBenchResult result;
  result.dispatch = attention_dispatch_name(config.tokens, config.head_dim, config.f16_kv);
  result.tokens = config.tokens;
  result.start_position = config.start_position;
  result.capacity_tokens = capacity_tokens;
  result.key_count = key_count;
  result.heads = config.heads;
  result.kv_heads = config.kv_heads;
  result.head_dim = config.head_dim;
  result.warmup_iterations = config.warmup_iterations;
  result.timed_iterations = config.timed_iterations;
  result.cache_values = static_cast<std::uint64_t>(cache_values);
  result.output_values_per_iteration = static_cast<std::uint64_t>(query_values);
  result.total_seconds = total_seconds;
  result.average_milliseconds = total_seconds * 1000.0 / timed;
  result.token_iterations_per_second = static_cast<double>(config.tokens) * timed / total_seconds;
  result.output_megavalues_per_second =
    static_cast<double>(query_values) * timed / (total_seconds * 1000000.0);
  result.sample_checksum = checksum.value();
  result.f16_kv = config.f16_kv;
  return result;
}

// format_qwen35_attention_bench_result (qwen35_runtime.cpp:5214-5236).
inline std::string format_attention_bench_result(const AttentionBenchResult& result) {
  std::ostringstream output;
  output << "Qwen3.5 HIP attention bench: ok\n";
  output << "Dispatch: " << result.dispatch << '\n';
  output << "KV cache: " << (result.f16_kv ? "f16" : "f32") << '\n';
  output << "Shape: tokens=" << result.tokens << ", start_position=" << result.start_position
         << ", key_count=" << result.key_count << ", capacity_tokens=" << result.capacity_tokens
         << ", heads=" << result.heads << ", kv_heads=" << result.kv_heads
         << ", head_dim=" << result.head_dim << '\n';
  output << "Iterations: warmup=" << result.warmup_iterations
         << ", timed=" << result.timed_iterations << '\n';
  output << "Cache values: " << result.cache_values << '\n';
  output << "Output values/iter: " << result.output_values_per_iteration << '\n';
  output << "Total seconds: " << result.total_seconds << '\n';
  output << "Average ms/iter: " << result.average_milliseconds << '\n';
  output << "Token-iterations/s: " << result.token_iterations_per_second << '\n';
  output << "Output Mvalues/s: " << result.output_megavalues_per_second << '\n';
  output << "Sample checksum: " << result.sample_checksum << '\n';
  return output.str();
}

}  // namespace qwen35
}  // namespace kraken
