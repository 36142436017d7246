// Drives the Qwen3.5 plan and layer drivers (include/kraken/qwen35_plan.hpp,
// include/kraken/qwen35_layers.hpp) for tests/test_qwen35_driver.py.
//
//   qwen35_driver_check plan
//       No GPU needed.  Prints the execution plan of Qwen3.5-0.8B for the
//       reference smoke test's request (11000 prompt tokens, chunks of 512) as
//       key=value lines and the formatted summary, the Status of the plan's
//       argument checks, and the layer walk of the decode loop.
//   qwen35_driver_check linear <dir> <reference|fused>
//   qwen35_driver_check full <dir> <reference|fused>
//       On a GPU.  Reads the chunk's projection outputs, weights and initial
//       caches from raw files in <dir> (written by the test), runs one layer
//       driver on the 0.8B plan and writes the output and the final caches
//       back to <dir>.
//   qwen35_driver_check gguf-info <file.gguf>
//       No GPU needed.  Parses a GGUF file and prints its header, tensor table
//       and metadata as lines, or "error <message>".
//   qwen35_driver_check decode <model.gguf> <outdir> <first_token> <steps> [trace] [reference]
//       On a GPU.  Loads a Qwen3.5-0.8B-shaped GGUF (include/kraken/gguf.hpp),
//       uploads its tensors, runs the greedy decode loop
//       (include/kraken/qwen35_decode.hpp) from position 0 and writes the
//       generated tokens (tokens.i32) to <outdir>; with `reference`, the
//       reference's separate ops instead of the fused GEMVs, and also the last
//       step's LM-head input (normed.f32); with `trace`, every layer's output
//       hidden state (hidden_trace.f32).
//   qwen35_driver_check prefill <model.gguf> <outdir> <prompt_tokens> <chunk_tokens> <steps>
//                               [trace] [reference]
//       On a GPU.  The same model: chunked prefill of a deterministic prompt
//       (include/kraken/qwen35_prefill.hpp), then greedy decode from the
//       prompt's end; writes prompt.i32 and tokens.i32, and with `trace` the
//       sampled hidden rows after every layer of every chunk and step.
// Exits non-zero on the first failure.
#include <algorithm>
#include <array>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iterator>
#include <memory>
#include <string>
#include <vector>

#include "kraken/gguf.hpp"
#include "kraken/qwen35_bench.hpp"
#include "kraken/qwen35_decode.hpp"
#include "kraken/qwen35_layers.hpp"
#include "kraken/qwen35_prefill.hpp"

using kraken::hip::HipBuffer;
using kraken::hip::HipContext;
using kraken::hip::Status;
namespace q35 = kraken::qwen35;

namespace {

const char* code_name(kraken::hip::StatusCode c) {
  switch (c) {
    case kraken::hip::StatusCode::ok:
      return "ok";
    case kraken::hip::StatusCode::invalid_argument:
      return "invalid_argument";
    case kraken::hip::StatusCode::unavailable:
      return "unavailable";
    default:
      return "internal_error";
  }
}

const char* kind_name(q35::LayerKind k) {
  switch (k) {
    case q35::LayerKind::full_attention:
      return "full_attention";
    case q35::LayerKind::linear_attention:
      return "linear_attention";
    default:
      return "mtp";
  }
}

void print_status(const char* label, const Status& s) {
  std::printf("status %s: %s %s\n", label, code_name(s.code()), s.message().c_str());
}

int run_plan() {
  q35::RuntimeOptions options;
  options.decode_tokens = 1;
  options.prefill_chunk_tokens = 512;
  const q35::ModelShape shape = q35::qwen35_0_8b_shape();
  auto plan = q35::build_execution_plan(shape, 11000, options);
  if (!plan.is_ok()) {
    print_status("plan", plan.status());
    return 1;
  }
  const q35::ExecutionPlan& p = plan.value();
  const q35::CachePlan& c = p.cache;
  std::printf("main_layers=%zu\n", p.main_layers);
  std::printf("full_attention_layers=%zu\n", c.full_attention_layers);
  std::printf("linear_attention_layers=%zu\n", c.linear_attention_layers);
  std::printf("kv_dim=%zu\n", c.kv_dim);
  std::printf("recurrent_r_elements_per_layer=%zu\n", c.recurrent_r_elements_per_layer);
  std::printf("recurrent_s_elements_per_layer=%zu\n", c.recurrent_s_elements_per_layer);
  std::printf("attention_capacity_tokens=%zu\n", c.attention_capacity_tokens);
  std::printf("chunk_count=%zu\n", p.prefill.chunk_count);
  std::printf("final_chunk_tokens=%zu\n", p.prefill.final_chunk_tokens);
  std::printf("output_only_last_token=%d\n", p.prefill.output_only_last_token ? 1 : 0);
  std::printf("kv_cache_bytes=%llu\n", (unsigned long long)c.kv_cache_bytes);
  std::printf("recurrent_r_cache_bytes=%llu\n", (unsigned long long)c.recurrent_r_cache_bytes);
  std::printf("recurrent_s_cache_bytes=%llu\n", (unsigned long long)c.recurrent_s_cache_bytes);
  std::printf("total_cache_bytes=%llu\n", (unsigned long long)c.total_cache_bytes);
  for (std::size_t i = 0; i < p.layer_kinds.size(); ++i) {
    std::printf("layer_kind %zu %s\n", i, kind_name(p.layer_kinds[i]));
  }
  std::printf("--- summary\n%s--- end\n", q35::format_execution_plan(p).c_str());

  // The plan's argument checks, in the reference's order.
  print_status("prompt_zero", q35::build_execution_plan(shape, 0, options).status());
  q35::RuntimeOptions bad = options;
  bad.prefill_chunk_tokens = 0;
  print_status("chunk_zero", q35::build_execution_plan(shape, 8, bad).status());
  bad = options;
  bad.sequence_slots = 0;
  print_status("slots_zero", q35::build_execution_plan(shape, 8, bad).status());
  q35::ModelShape s2 = shape;
  s2.hidden_size = 0;
  s2.head_dim = -1;
  print_status("hidden_zero", q35::build_execution_plan(s2, 8, options).status());
  s2 = shape;
  s2.head_dim = -1;
  print_status("head_dim_negative", q35::build_execution_plan(s2, 8, options).status());
  s2 = shape;
  s2.linear_inner_size = 2047;
  print_status("inner_indivisible", q35::build_execution_plan(s2, 8, options).status());
  s2 = shape;
  s2.layer_kinds.resize(23);
  print_status("kinds_short", q35::build_execution_plan(s2, 8, options).status());
  bad = options;
  bad.context_tokens = (std::size_t)1 << 62;
  print_status("kv_overflow", q35::build_execution_plan(shape, 8, bad).status());

  // Options that change every cache term.
  q35::RuntimeOptions o2;
  o2.context_tokens = 262144;
  o2.decode_tokens = 64;
  o2.prefill_chunk_tokens = 1000;
  o2.sequence_slots = 2;
  o2.recurrent_snapshot_count = 3;
  o2.kv_cache_f16 = false;
  o2.output_all_prompt_logits = true;
  auto plan2 = q35::build_execution_plan(shape, 3000, o2);
  if (!plan2.is_ok()) {
    print_status("plan2", plan2.status());
    return 1;
  }
  std::printf("--- summary2\n%s--- end\n", q35::format_execution_plan(plan2.value()).c_str());

  // A model with one MTP layer past the main ones: counted in neither cache.
  q35::ModelShape s3 = shape;
  s3.total_layer_count = 25;
  s3.layer_kinds = q35::default_layer_kinds(24, 25);
  auto plan3 = q35::build_execution_plan(s3, 16, options);
  std::printf("mtp_model: %s main=%zu total=%zu full=%zu linear=%zu\n",
              code_name(plan3.status().code()), plan3.value().main_layers,
              plan3.value().total_layers, plan3.value().cache.full_attention_layers,
              plan3.value().cache.linear_attention_layers);

  // The decode loop's layer walk.
  const Status walk = q35::for_each_main_layer(
    p, [](std::size_t i, q35::LayerKind k, std::size_t kind_index) {
      std::printf("walk %zu %s %zu\n", i, kind_name(k), kind_index);
      return Status::ok();
    });
  print_status("walk", walk);
  q35::ExecutionPlan p4 = p;
  p4.layer_kinds[5] = q35::LayerKind::mtp;
  print_status("walk_mtp", q35::for_each_main_layer(p4, [](std::size_t, q35::LayerKind,
                                                           std::size_t) { return Status::ok(); }));
  q35::ExecutionPlan p5 = p;
  p5.layer_kinds[4] = q35::LayerKind::full_attention;
  print_status("walk_count", q35::for_each_main_layer(p5, [](std::size_t, q35::LayerKind,
                                                             std::size_t) { return Status::ok(); }));
  std::printf("plan done\n");
  return 0;
}

template <typename T>
bool read_file(const std::string& path, std::vector<T>& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) {
    std::printf("FAIL cannot read %s\n", path.c_str());
    return false;
  }
  std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  out.resize(bytes.size() / sizeof(T));
  std::memcpy(out.data(), bytes.data(), out.size() * sizeof(T));
  return true;
}

template <typename T>
bool write_file(const std::string& path, const std::vector<T>& data) {
  std::ofstream f(path, std::ios::binary);
  f.write(reinterpret_cast<const char*>(data.data()), (std::streamsize)(data.size() * sizeof(T)));
  return (bool)f;
}

bool check(const Status& s, const char* what) {
  if (!s.is_ok()) {
    std::printf("FAIL %s: %s %s\n", what, code_name(s.code()), s.message().c_str());
    return false;
  }
  return true;
}

// Device buffer holding `host`.
template <typename T>
bool upload(const HipContext& ctx, const std::vector<T>& host, HipBuffer& out) {
  auto b = ctx.make_buffer(host.size() * sizeof(T));
  if (!check(b.status(), "make_buffer")) {
    return false;
  }
  out = std::move(b.value());
  return check(ctx.copy_to_buffer(out, host.data(), host.size() * sizeof(T)), "upload");
}

template <typename T>
bool download(const HipContext& ctx, const HipBuffer& b, std::vector<T>& host) {
  host.resize(b.byte_size() / sizeof(T));
  return check(ctx.copy_from_buffer(b, host.data(), host.size() * sizeof(T)), "download");
}

// meta.txt: whitespace-separated integers.
bool read_meta(const std::string& dir, std::vector<long long>& meta) {
  std::ifstream f(dir + "/meta.txt");
  long long v;
  while (f >> v) {
    meta.push_back(v);
  }
  return !meta.empty();
}

int run_linear(const std::string& dir, q35::OpOrder order) {
  std::vector<long long> meta;  // tokens, linear_layer
  if (!read_meta(dir, meta) || meta.size() < 2) {
    std::printf("FAIL meta\n");
    return 1;
  }
  const std::size_t tokens = (std::size_t)meta[0];
  const std::size_t layer = (std::size_t)meta[1];
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  q35::RuntimeOptions options;
  auto plan = q35::build_execution_plan(q35::qwen35_0_8b_shape(), tokens, options);
  if (!check(plan.status(), "plan")) {
    return 1;
  }
  auto cache = q35::allocate_device_cache(ctx, plan.value());
  if (!check(cache.status(), "allocate_device_cache")) {
    return 1;
  }
  std::vector<float> qkv, z, beta, alpha, conv1d, dt_bias, ssm_a, norm, r0, s0;
  const std::pair<const char*, std::vector<float>*> inputs[] = {
    {"qkv", &qkv},         {"z", &z},         {"beta", &beta}, {"alpha", &alpha},
    {"conv1d", &conv1d},   {"dt_bias", &dt_bias}, {"ssm_a", &ssm_a},
    {"ssm_norm", &norm},   {"r0", &r0},       {"s0", &s0},
  };
  for (const auto& in : inputs) {
    if (!read_file(dir + "/" + in.first + ".f32", *in.second)) {
      return 1;
    }
  }
  HipBuffer qkv_b, z_b, beta_b, alpha_b, conv_b, dtb_b, a_b, norm_b;
  if (!upload(ctx, qkv, qkv_b) || !upload(ctx, z, z_b) || !upload(ctx, beta, beta_b) ||
      !upload(ctx, alpha, alpha_b) || !upload(ctx, conv1d, conv_b) ||
      !upload(ctx, dt_bias, dtb_b) || !upload(ctx, ssm_a, a_b) || !upload(ctx, norm, norm_b)) {
    return 1;
  }
  q35::DeviceCache& dc = cache.value();
  if (r0.size() * 4 != dc.recurrent_r_cache.byte_size() ||
      s0.size() * 4 != dc.recurrent_s_cache.byte_size()) {
    std::printf("FAIL initial cache sizes\n");
    return 1;
  }
  if (!check(ctx.copy_to_buffer(dc.recurrent_r_cache, r0.data(), r0.size() * 4), "r0") ||
      !check(ctx.copy_to_buffer(dc.recurrent_s_cache, s0.data(), s0.size() * 4), "s0")) {
    return 1;
  }
  auto out = ctx.make_buffer(tokens * plan.value().linear_inner_size * 4);
  if (!check(out.status(), "output")) {
    return 1;
  }
  q35::LinearAttentionWeights w{&conv_b, &dtb_b, &a_b, &norm_b};
  q35::LayerWorkspace ws;
  if (!check(q35::run_linear_attention_chunk(ctx, plan.value(), dc, w, layer, 0, qkv_b, z_b,
                                             beta_b, alpha_b, tokens, 1e-6f, order, ws,
                                             out.value()),
             "run_linear_attention_chunk")) {
    return 1;
  }
  std::vector<float> y, r1, s1;
  if (!download(ctx, out.value(), y) || !download(ctx, dc.recurrent_r_cache, r1) ||
      !download(ctx, dc.recurrent_s_cache, s1)) {
    return 1;
  }
  write_file(dir + "/out.f32", y);
  write_file(dir + "/r1.f32", r1);
  write_file(dir + "/s1.f32", s1);
  std::printf("linear done\n");
  return 0;
}

int run_full(const std::string& dir, q35::OpOrder order) {
  std::vector<long long> meta;  // tokens, start_position, attention_layer, capacity
  if (!read_meta(dir, meta) || meta.size() < 4) {
    std::printf("FAIL meta\n");
    return 1;
  }
  const std::size_t tokens = (std::size_t)meta[0];
  const std::size_t start = (std::size_t)meta[1];
  const std::size_t layer = (std::size_t)meta[2];
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  q35::RuntimeOptions options;
  options.context_tokens = (std::size_t)meta[3];
  auto plan = q35::build_execution_plan(q35::qwen35_0_8b_shape(), start + tokens, options);
  if (!check(plan.status(), "plan")) {
    return 1;
  }
  auto cache = q35::allocate_device_cache(ctx, plan.value());
  if (!check(cache.status(), "allocate_device_cache")) {
    return 1;
  }
  std::vector<float> qg, key, value, qn, kn;
  std::vector<std::uint16_t> kc0, vc0;
  if (!read_file(dir + "/qg.f32", qg) || !read_file(dir + "/key.f32", key) ||
      !read_file(dir + "/value.f32", value) || !read_file(dir + "/q_norm.f32", qn) ||
      !read_file(dir + "/k_norm.f32", kn) || !read_file(dir + "/kc0.u16", kc0) ||
      !read_file(dir + "/vc0.u16", vc0)) {
    return 1;
  }
  q35::DeviceCache& dc = cache.value();
  if (kc0.size() * 2 != dc.key_cache.byte_size() || vc0.size() * 2 != dc.value_cache.byte_size()) {
    std::printf("FAIL initial cache sizes\n");
    return 1;
  }
  if (!check(ctx.copy_to_buffer(dc.key_cache, kc0.data(), kc0.size() * 2), "kc0") ||
      !check(ctx.copy_to_buffer(dc.value_cache, vc0.data(), vc0.size() * 2), "vc0")) {
    return 1;
  }
  HipBuffer qg_b, key_b, value_b, qn_b, kn_b;
  if (!upload(ctx, qg, qg_b) || !upload(ctx, key, key_b) || !upload(ctx, value, value_b) ||
      !upload(ctx, qn, qn_b) || !upload(ctx, kn, kn_b)) {
    return 1;
  }
  const q35::ExecutionPlan& p = plan.value();
  auto out = ctx.make_buffer(tokens * p.attention_heads * p.head_dim * 4);
  if (!check(out.status(), "output")) {
    return 1;
  }
  q35::FullAttentionWeights w{&qn_b, &kn_b};
  q35::LayerWorkspace ws;
  // Qwen3.5 MRoPE sections and rope theta (qwen3-5-0-8b-llama-cpp-ops.md:64).
  const std::array<std::size_t, 4> sections{11, 11, 10, 0};
  if (!check(q35::run_full_attention_chunk(ctx, p, dc, w, layer, qg_b, key_b, value_b, tokens,
                                           start, start, sections, 1e7f, 1e-6f, nullptr, order,
                                           ws, out.value()),
             "run_full_attention_chunk")) {
    return 1;
  }
  std::vector<float> y;
  std::vector<std::uint16_t> kc1, vc1;
  if (!download(ctx, out.value(), y) || !download(ctx, dc.key_cache, kc1) ||
      !download(ctx, dc.value_cache, vc1)) {
    return 1;
  }
  write_file(dir + "/out.f32", y);
  write_file(dir + "/kc1.u16", kc1);
  write_file(dir + "/vc1.u16", vc1);
  std::printf("full done\n");
  return 0;
}

}  // namespace

// bench-matmul <model.gguf|dir> <tensor> <tokens> <warmup> <timed>
// bench-gdn <tokens> <key_heads> <value_heads> <head_dim> <warmup> <timed>
// bench-attention <tokens> <start> <capacity> <heads> <kv_heads> <head_dim> <warmup> <timed> <f16>
// Prints the formatted result, or "error <code>: <message>" (exit 1).
int run_bench(const std::string& mode, int argc, char** argv) {
  auto arg = [&](int i) { return (std::size_t)std::strtoull(argv[i], nullptr, 10); };
  auto fail = [](const kraken::hip::Status& s) {
    std::printf("error %d: %s\n", (int)s.code(), s.message().c_str());
    return 1;
  };
  if (mode == "bench-matmul" && argc >= 7) {
    q35::MatmulBenchConfig c;
    c.model_path = argv[2];
    c.tensor_name = argv[3];
    c.tokens = arg(4);
    c.warmup_iterations = arg(5);
    c.timed_iterations = arg(6);
    auto r = q35::benchmark_matmul(c);
    if (!r.is_ok()) {
      return fail(r.status());
    }
    std::printf("%s", q35::format_matmul_bench_result(r.value()).c_str());
    std::printf("checksum_exact %.17g\n", r.value().sample_checksum);
    return 0;
  }
  if (mode == "bench-gdn" && argc >= 8) {
    q35::GdnBenchConfig c;
    c.tokens = arg(2);
    c.key_heads = arg(3);
    c.value_heads = arg(4);
    c.head_dim = arg(5);
    c.warmup_iterations = arg(6);
    c.timed_iterations = arg(7);
    auto r = q35::benchmark_gdn(c);
    if (!r.is_ok()) {
      return fail(r.status());
    }
    std::printf("%s", q35::format_gdn_bench_result(r.value()).c_str());
    std::printf("checksum_exact %.17g\n", r.value().sample_checksum);
    return 0;
  }
  if (mode == "bench-attention" && argc >= 11) {
    q35::AttentionBenchConfig c;
    c.tokens = arg(2);
    c.start_position = arg(3);
    c.capacity_tokens = arg(4);
    c.heads = arg(5);
    c.kv_heads = arg(6);
    c.head_dim = arg(7);
    c.warmup_iterations = arg(8);
    c.timed_iterations = arg(9);
    c.f16_kv = arg(10) != 0;
    auto r = q35::benchmark_attention(c);
    if (!r.is_ok()) {
      return fail(r.status());
    }
    std::printf("%s", q35::format_attention_bench_result(r.value()).c_str());
    std::printf("checksum_exact %.17g\n", r.value().sample_checksum);
    return 0;
  }
  std::printf("usage: see run_bench\n");
  return 2;
}

// Device copies of a GGUF's tensors, by name.
class DeviceTensors {
 public:
  DeviceTensors(const HipContext& ctx, const kraken::gguf::File& f,
                const kraken::gguf::MappedData& m)
      : ctx_(ctx), file_(f), map_(m) {}

  // The tensor `name` as a projection / embedding (2-D, GGUF shape {cols, rows}),
  // or a vector (1-D, rows = 1); missing or failing loads print and return false.
  bool get(const std::string& name, q35::Tensor& out) {
    const kraken::gguf::TensorInfo* t = kraken::gguf::find_tensor(file_, name);
    if (t == nullptr) {
      std::printf("FAIL missing tensor %s\n", name.c_str());
      return false;
    }
    auto bytes = map_.tensor_bytes(*t);
    if (!check(bytes.status(), name.c_str())) {
      return false;
    }
    auto b = ctx_.make_buffer(bytes.value().second);
    if (!check(b.status(), name.c_str()) ||
        !check(ctx_.copy_to_buffer(b.value(), bytes.value().first, bytes.value().second),
               name.c_str())) {
      return false;
    }
    owned_.push_back(std::make_unique<HipBuffer>(std::move(b.value())));
    out.buffer = owned_.back().get();
    out.type = static_cast<q35::TensorType>(t->type);
    out.cols = (std::size_t)t->shape[0];
    out.rows = t->shape.size() > 1 ? (std::size_t)t->shape[1] : 1;
    return true;
  }
  bool vec(const std::string& name, const HipBuffer*& out) {
    q35::Tensor t;
    if (!get(name, t)) {
      return false;
    }
    out = t.buffer;
    return true;
  }

 private:
  const HipContext& ctx_;
  const kraken::gguf::File& file_;
  const kraken::gguf::MappedData& map_;
  std::vector<std::unique_ptr<HipBuffer>> owned_;
};

// A Qwen3.5-0.8B-shaped GGUF on the device: the file, its mapping, the
// uploaded tensors and the weights table of the plan.
struct LoadedModel {
  kraken::gguf::File file;
  std::unique_ptr<kraken::gguf::MappedData> map;
  std::unique_ptr<DeviceTensors> tensors;
  q35::ModelWeights weights;
};

bool load_gguf_model(const HipContext& ctx, const std::string& path, const q35::ExecutionPlan& plan,
                     LoadedModel& m) {
  auto file = kraken::gguf::read_file(path);
  if (!check(file.status(), "read GGUF")) {
    return false;
  }
  m.file = std::move(file.value());
  auto map = kraken::gguf::MappedData::open(m.file);
  if (!check(map.status(), "map GGUF")) {
    return false;
  }
  m.map = std::make_unique<kraken::gguf::MappedData>(std::move(map.value()));
  const q35::ModelShape shape = q35::qwen35_0_8b_shape();
  auto blocks = kraken::gguf::get_i64(m.file, "qwen35.block_count");
  auto width = kraken::gguf::get_i64(m.file, "qwen35.embedding_length");
  if (!check(blocks.status(), "block_count") || !check(width.status(), "embedding_length") ||
      blocks.value() != shape.total_layer_count || width.value() != shape.hidden_size) {
    std::printf("FAIL GGUF is not Qwen3.5-0.8B shaped\n");
    return false;
  }
  m.tensors = std::make_unique<DeviceTensors>(ctx, m.file, *m.map);
  DeviceTensors& dt = *m.tensors;
  q35::ModelWeights& w = m.weights;
  if (!dt.get("token_embd.weight", w.token_embd) ||
      !dt.vec("output_norm.weight", w.output_norm)) {
    return false;
  }
  // output.weight absent: the LM head is tied to token_embd (qwen35.cpp:45-52
  // of llama.cpp, as the reference's loader does).
  if (kraken::gguf::find_tensor(m.file, "output.weight") != nullptr) {
    if (!dt.get("output.weight", w.output)) {
      return false;
    }
  } else {
    w.output = w.token_embd;
  }
  w.layers.resize(plan.main_layers);
  for (std::size_t i = 0; i < plan.main_layers; ++i) {
    const std::string p = "blk." + std::to_string(i) + ".";
    q35::DecoderLayerWeights& l = w.layers[i];
    bool ok = dt.vec(p + "attn_norm.weight", l.attn_norm) &&
              dt.vec(p + "post_attention_norm.weight", l.post_attention_norm) &&
              dt.get(p + "ffn_gate.weight", l.ffn_gate) && dt.get(p + "ffn_up.weight", l.ffn_up) &&
              dt.get(p + "ffn_down.weight", l.ffn_down);
    if (ok && plan.layer_kinds[i] == q35::LayerKind::linear_attention) {
      ok = dt.get(p + "attn_qkv.weight", l.qkv) && dt.get(p + "attn_gate.weight", l.gate) &&
           dt.get(p + "ssm_beta.weight", l.beta) && dt.get(p + "ssm_alpha.weight", l.alpha) &&
           dt.get(p + "ssm_out.weight", l.ssm_out) &&
           dt.vec(p + "ssm_conv1d.weight", l.linear.conv1d) &&
           dt.vec(p + "ssm_dt.bias", l.linear.dt_bias) && dt.vec(p + "ssm_a", l.linear.ssm_a) &&
           dt.vec(p + "ssm_norm.weight", l.linear.ssm_norm);
    } else if (ok) {
      ok = dt.get(p + "attn_q.weight", l.q) && dt.get(p + "attn_k.weight", l.k) &&
           dt.get(p + "attn_v.weight", l.v) && dt.get(p + "attn_output.weight", l.output) &&
           dt.vec(p + "attn_q_norm.weight", l.full.q_norm) &&
           dt.vec(p + "attn_k_norm.weight", l.full.k_norm);
    }
    if (!ok) {
      return false;
    }
  }
  return true;
}

int run_decode(const std::string& path, const std::string& out_dir, std::int32_t first_token,
               std::size_t steps, bool trace, q35::OpOrder order) {
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  q35::RuntimeOptions options;
  options.context_tokens = steps + 1;
  auto plan = q35::build_execution_plan(q35::qwen35_0_8b_shape(), steps, options);
  if (!check(plan.status(), "plan")) {
    return 1;
  }
  auto cache = q35::allocate_device_cache(ctx, plan.value());
  if (!check(cache.status(), "allocate_device_cache")) {
    return 1;
  }
  LoadedModel model;
  if (!load_gguf_model(ctx, path, plan.value(), model)) {
    return 1;
  }
  const q35::ModelWeights& w = model.weights;
  q35::DecodeScratch scratch;
  // With `trace`, every layer's output hidden state of every step is appended
  // to hidden_trace.f32 (steps x layers x hidden).
  std::vector<float> trace_rows;
  const q35::LayerHook hook = [&](std::size_t, const HipBuffer& hidden) {
    std::vector<float> row(plan.value().hidden_size);
    const Status st = ctx.copy_from_buffer(hidden, row.data(), row.size() * sizeof(float));
    trace_rows.insert(trace_rows.end(), row.begin(), row.end());
    return st;
  };
  auto tokens = q35::greedy_decode(ctx, plan.value(), cache.value(), w, scratch, first_token, 0,
                                   steps, trace ? &hook : nullptr, order);
  if (trace && !write_file(out_dir + "/hidden_trace.f32", trace_rows)) {
    std::printf("FAIL write trace\n");
    return 1;
  }
  if (!check(tokens.status(), "greedy_decode")) {
    return 1;
  }
  if (!write_file(out_dir + "/tokens.i32", tokens.value())) {
    std::printf("FAIL write outputs\n");
    return 1;
  }
  if (order == q35::OpOrder::reference) {
    std::vector<float> normed(plan.value().hidden_size);
    if (!check(ctx.copy_from_buffer(scratch.normed, normed.data(), normed.size() * 4),
               "normed") ||
        !write_file(out_dir + "/normed.f32", normed)) {
      return 1;
    }
  }
  std::printf("decode done:");
  for (const std::int32_t t : tokens.value()) {
    std::printf(" %d", t);
  }
  std::printf("\n");
  return 0;
}

// prefill <model.gguf> <outdir> <prompt_tokens> <chunk_tokens> <steps> [trace] [reference]:
// chunked prefill of a deterministic prompt (token i = (7919 i + 11) mod vocab,
// written to prompt.i32), then greedy decode; the generated tokens go to
// tokens.i32 (the prefill's token first).  With `trace`, the hidden state after
// every layer of every chunk is sampled at the chunk's rows 0, tokens / 2 and
// tokens - 1 (prefill_trace.f32, [chunk][layer][3][hidden]) and after every
// layer of every decode step (hidden_trace.f32, [step][layer][hidden]).
int run_prefill(const std::string& path, const std::string& out_dir, std::size_t prompt_tokens,
                std::size_t chunk_tokens, std::size_t steps, bool trace, q35::OpOrder order) {
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  q35::RuntimeOptions options;
  options.prefill_chunk_tokens = chunk_tokens;
  options.decode_tokens = steps;
  auto plan = q35::build_execution_plan(q35::qwen35_0_8b_shape(), prompt_tokens, options);
  if (!check(plan.status(), "plan")) {
    return 1;
  }
  auto cache = q35::allocate_device_cache(ctx, plan.value());
  if (!check(cache.status(), "allocate_device_cache")) {
    return 1;
  }
  LoadedModel model;
  if (!load_gguf_model(ctx, path, plan.value(), model)) {
    return 1;
  }
  const q35::ModelWeights& w = model.weights;
  const std::size_t h = plan.value().hidden_size;
  std::vector<std::int32_t> prompt(prompt_tokens);
  for (std::size_t i = 0; i < prompt_tokens; ++i) {
    prompt[i] = (std::int32_t)((7919u * i + 11u) % w.token_embd.rows);
  }
  std::vector<float> prefill_rows;
  const q35::ChunkLayerHook chunk_hook = [&](std::size_t, const HipBuffer& hidden,
                                             std::size_t, std::size_t tokens) {
    std::vector<float> all(tokens * h);
    const Status st = ctx.copy_from_buffer(hidden, all.data(), all.size() * sizeof(float));
    for (const std::size_t r : {std::size_t{0}, tokens / 2, tokens - 1}) {
      prefill_rows.insert(prefill_rows.end(), all.begin() + r * h, all.begin() + (r + 1) * h);
    }
    return st;
  };
  std::vector<float> decode_rows;
  const q35::LayerHook step_hook = [&](std::size_t, const HipBuffer& hidden) {
    std::vector<float> row(h);
    const Status st = ctx.copy_from_buffer(hidden, row.data(), row.size() * sizeof(float));
    decode_rows.insert(decode_rows.end(), row.begin(), row.end());
    return st;
  };
  q35::PrefillScratch ps;
  q35::DecodeScratch ds;
  const auto t0 = std::chrono::steady_clock::now();
  auto first = q35::prefill_prompt(ctx, plan.value(), cache.value(), w, ps, prompt,
                                   trace ? &chunk_hook : nullptr, order);
  const double prefill_ms =
    std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  if (!check(first.status(), "prefill_prompt")) {
    return 1;
  }
  std::vector<std::int32_t> tokens{first.value()};
  if (steps > 1) {
    auto rest = q35::greedy_decode(ctx, plan.value(), cache.value(), w, ds, first.value(),
                                   prompt_tokens, steps - 1, trace ? &step_hook : nullptr, order);
    if (!check(rest.status(), "greedy_decode")) {
      return 1;
    }
    tokens.insert(tokens.end(), rest.value().begin(), rest.value().end());
  }
  if (!write_file(out_dir + "/prompt.i32", prompt) ||
      !write_file(out_dir + "/tokens.i32", tokens) ||
      (trace && (!write_file(out_dir + "/prefill_trace.f32", prefill_rows) ||
                 !write_file(out_dir + "/hidden_trace.f32", decode_rows)))) {
    std::printf("FAIL write outputs\n");
    return 1;
  }
  std::printf("prefill done: chunks=%zu prefill_ms=%.3f tokens:", plan.value().prefill.chunk_count,
              prefill_ms);
  for (const std::int32_t t : tokens) {
    std::printf(" %d", t);
  }
  std::printf("\n");
  return 0;
}

int run_gguf_info(const std::string& path) {
  auto f = kraken::gguf::read_file(path);
  if (!f.is_ok()) {
    std::printf("error %s\n", f.status().message().c_str());
    return 1;
  }
  const kraken::gguf::File& g = f.value();
  std::printf("version=%u tensors=%llu metadata=%llu alignment=%llu data_offset=%llu\n",
              g.version, (unsigned long long)g.tensor_count,
              (unsigned long long)g.metadata_count, (unsigned long long)g.alignment,
              (unsigned long long)g.data_offset);
  auto map = kraken::gguf::MappedData::open(g);
  for (const auto& t : g.tensors) {
    std::string shape;
    for (const auto d : t.shape) {
      shape += (shape.empty() ? "" : ",") + std::to_string(d);
    }
    unsigned long long sum = 0;  // byte sum of the tensor's data, read through the mapping
    if (map.is_ok()) {
      auto bytes = map.value().tensor_bytes(t);
      if (bytes.is_ok()) {
        for (std::size_t i = 0; i < bytes.value().second; ++i) {
          sum += bytes.value().first[i];
        }
      }
    }
    std::printf("tensor %s type=%u shape=%s offset=%llu abs=%llu bytes=%llu sum=%llu\n",
                t.name.c_str(), t.type, shape.c_str(), (unsigned long long)t.offset,
                (unsigned long long)t.absolute_offset, (unsigned long long)t.byte_size, sum);
  }
  std::vector<std::string> keys;
  for (const auto& kv : g.metadata) {
    keys.push_back(kv.first);
  }
  std::sort(keys.begin(), keys.end());
  for (const auto& k : keys) {
    const auto& v = g.metadata.at(k);
    std::string val;
    if (v.kind == kraken::gguf::ValueKind::array) {
      val = "array[" + std::to_string(v.count) + "]";
      if (!v.sa.empty()) val += " first=" + v.sa.front();
      if (!v.ia.empty()) val += " first=" + std::to_string(v.ia.front());
      if (!v.ua.empty()) val += " first=" + std::to_string(v.ua.front());
    } else if (v.kind == kraken::gguf::ValueKind::string) {
      val = v.s;
    } else {
      auto i = kraken::gguf::get_i64(g, k);
      auto d = kraken::gguf::get_f64(g, k);
      val = i.is_ok() ? std::to_string(i.value())
                      : (d.is_ok() ? std::to_string(d.value()) : (v.b ? "true" : "false"));
    }
    std::printf("meta %s kind=%u %s\n", k.c_str(), (unsigned)v.kind, val.c_str());
  }
  return 0;
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "plan";
  if (mode == "plan") {
    return run_plan();
  }
  if (mode.rfind("bench-", 0) == 0) {
    return run_bench(mode, argc, argv);
  }
  if (mode == "gguf-info" && argc >= 3) {
    return run_gguf_info(argv[2]);
  }
  if (mode == "decode" && argc >= 6) {
    bool trace = false;
    q35::OpOrder order = q35::OpOrder::fused;
    for (int i = 6; i < argc; ++i) {
      trace = trace || std::string(argv[i]) == "trace";
      order = std::string(argv[i]) == "reference" ? q35::OpOrder::reference : order;
    }
    return run_decode(argv[2], argv[3], (std::int32_t)std::stol(argv[4]),
                      (std::size_t)std::stoul(argv[5]), trace, order);
  }
  if (mode == "prefill" && argc >= 7) {
    bool trace = false;
    q35::OpOrder order = q35::OpOrder::fused;
    for (int i = 7; i < argc; ++i) {
      trace = trace || std::string(argv[i]) == "trace";
      order = std::string(argv[i]) == "reference" ? q35::OpOrder::reference : order;
    }
    return run_prefill(argv[2], argv[3], (std::size_t)std::stoul(argv[4]),
                       (std::size_t)std::stoul(argv[5]), (std::size_t)std::stoul(argv[6]), trace,
                       order);
  }
  if (argc < 4) {
    std::printf("usage: qwen35_driver_check plan | linear <dir> <order> | full <dir> <order> | "
                "decode <model.gguf> <outdir> <first_token> <steps> | "
                "prefill <model.gguf> <outdir> <prompt> <chunk> <steps>\n");
    return 2;
  }
  const q35::OpOrder order =
    std::string(argv[3]) == "fused" ? q35::OpOrder::fused : q35::OpOrder::reference;
  if (mode == "linear") {
    return run_linear(argv[2], order);
  }
  if (mode == "full") {
    return run_full(argv[2], order);
  }
  std::printf("unknown mode %s\n", mode.c_str());
  return 2;
}
