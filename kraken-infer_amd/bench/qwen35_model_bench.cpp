// Whole-model timings of the MI355X Qwen3.5 path on synthetic Qwen3.5-0.8B
// weights, for bench.py (no counterpart in the reference, whose benches time
// single ops: qwen35_runtime.cpp:4558-5236).  Each mode prints one line of
// key=value fields.
//
//   qwen35_model_bench decode <warmup> <steps> [reference]
//       Greedy decode (include/kraken/qwen35_decode.hpp) of `steps` tokens after
//       `warmup` tokens: one graph batch and one host wait per token, the next
//       token kept on the device; the fused op order unless `reference`.
//   qwen35_model_bench prefill <prompt_tokens> <chunk_tokens> [reference]
//       Chunked prefill of the whole model (include/kraken/qwen35_prefill.hpp):
//       one untimed pass, then one timed pass over the same prompt (one graph
//       batch and one host wait per chunk), ending with the greedy LM head.
//   qwen35_model_bench prefix-store
//       Commit and restore of 1024-token blocks of the Qwen3.5-0.8B cache in the
//       prompt prefix store (include/kraken/qwen35_prefix_store.hpp).
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "kraken/qwen35_decode.hpp"
#include "kraken/qwen35_prefill.hpp"
#include "kraken/qwen35_prefix_store.hpp"

using kraken::hip::HipBuffer;
using kraken::hip::HipContext;
using kraken::hip::Status;
namespace q35 = kraken::qwen35;

namespace {

bool check(const Status& s, const char* what) {
  if (!s.is_ok()) {
    std::printf("FAIL %s: %s\n", what, s.message().c_str());
    return false;
  }
  return true;
}

// Synthetic Qwen3.5-0.8B weights on the device: random K-quant blocks with f16
// scales chosen so that weights are a few hundredths, f32 norms near 1.
class SyntheticModel {
 public:
  explicit SyntheticModel(const HipContext& ctx) : ctx_(ctx) {}
  std::uint64_t bytes() const { return bytes_; }

  bool quant(q35::TensorType type, std::size_t rows, std::size_t cols, q35::Tensor& out) {
    const std::size_t nb =
      type == q35::TensorType::q4_k ? 144 : (type == q35::TensorType::q5_k ? 176 : 210);
    const std::size_t blocks = rows * cols / 256;
    std::vector<std::uint8_t> data(blocks * nb);
    for (auto& b : data) {
      b = (std::uint8_t)(next() >> 56);
    }
    const float d = type == q35::TensorType::q4_k ? 1.5e-4f
                                                   : (type == q35::TensorType::q5_k ? 8e-5f : 4e-5f);
    for (std::size_t i = 0; i < blocks; ++i) {
      std::uint8_t* blk = data.data() + i * nb;
      const std::uint16_t dh = half_bits(d * (0.5f + unit()));
      if (type == q35::TensorType::q6_k) {
        std::memcpy(blk + 208, &dh, 2);
      } else {
        const std::uint16_t mh = half_bits(1e-3f * unit());
        std::memcpy(blk, &dh, 2);
        std::memcpy(blk + 2, &mh, 2);
      }
    }
    if (!upload(data, out.buffer)) {
      return false;
    }
    out.type = type;
    out.rows = rows;
    out.cols = cols;
    return true;
  }
  bool vec(std::size_t n, float base, float spread, const HipBuffer*& out) {
    std::vector<float> v(n);
    for (auto& x : v) {
      x = base + spread * (2.0f * unit() - 1.0f);
    }
    return upload(v, out);
  }

  // Every tensor of the 0.8B plan's main layers, the tied Q6_K embedding / LM
  // head and the output norm.
  bool build(const q35::ExecutionPlan& plan, q35::ModelWeights& w) {
    using TT = q35::TensorType;
    const std::size_t h = plan.hidden_size, ffn = 3584;
    bool ok = quant(TT::q6_k, 248320, h, w.token_embd) && vec(h, 1.0f, 0.1f, w.output_norm);
    w.output = w.token_embd;
    w.layers.resize(plan.main_layers);
    for (std::size_t i = 0; ok && i < w.layers.size(); ++i) {
      q35::DecoderLayerWeights& l = w.layers[i];
      ok = vec(h, 1.0f, 0.1f, l.attn_norm) && vec(h, 1.0f, 0.1f, l.post_attention_norm) &&
           quant(TT::q4_k, ffn, h, l.ffn_gate) && quant(TT::q4_k, ffn, h, l.ffn_up) &&
           quant(TT::q6_k, h, ffn, l.ffn_down);
      if (ok && plan.layer_kinds[i] == q35::LayerKind::linear_attention) {
        ok = quant(TT::q5_k, 6144, h, l.qkv) && quant(TT::q4_k, 2048, h, l.gate) &&
             quant(TT::q4_k, 16, h, l.beta) && quant(TT::q4_k, 16, h, l.alpha) &&
             quant(TT::q4_k, h, 2048, l.ssm_out) && vec(6144 * 4, 0.0f, 0.5f, l.linear.conv1d) &&
             vec(16, 0.0f, 0.5f, l.linear.dt_bias) && vec(16, -0.7f, 0.5f, l.linear.ssm_a) &&
             vec(128, 1.0f, 0.1f, l.linear.ssm_norm);
      } else if (ok) {
        ok = quant(TT::q4_k, 4096, h, l.q) && quant(TT::q4_k, 512, h, l.k) &&
             quant(TT::q6_k, 512, h, l.v) && quant(TT::q4_k, h, 2048, l.output) &&
             vec(256, 1.0f, 0.1f, l.full.q_norm) && vec(256, 1.0f, 0.1f, l.full.k_norm);
      }
    }
    return ok;
  }

 private:
  template <typename T>
  bool upload(const std::vector<T>& host, const HipBuffer*& out) {
    auto b = ctx_.make_buffer(host.size() * sizeof(T));
    if (!check(b.status(), "make_buffer") ||
        !check(ctx_.copy_to_buffer(b.value(), host.data(), host.size() * sizeof(T)), "upload")) {
      return false;
    }
    bytes_ += host.size() * sizeof(T);
    owned_.push_back(std::make_unique<HipBuffer>(std::move(b.value())));
    out = owned_.back().get();
    return true;
  }
  std::uint64_t next() {  // xorshift64*
    state_ ^= state_ >> 12;
    state_ ^= state_ << 25;
    state_ ^= state_ >> 27;
    return state_ * 0x2545F4914F6CDD1DULL;
  }
  float unit() { return (float)(next() >> 40) / (float)(1 << 24); }
  static std::uint16_t half_bits(float f) {  // small positive normal values only
    std::uint32_t x;
    std::memcpy(&x, &f, 4);
    const int e = (int)((x >> 23) & 0xFF) - 127 + 15;
    return (std::uint16_t)((e << 10) | ((x >> 13) & 0x3FF));
  }

  const HipContext& ctx_;
  std::vector<std::unique_ptr<HipBuffer>> owned_;
  std::uint64_t bytes_{0};
  std::uint64_t state_{0x9E3779B97F4A7C15ULL};
};

int run_decode(std::size_t warmup, std::size_t steps, q35::OpOrder order) {
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  q35::RuntimeOptions options;
  options.context_tokens = warmup + steps + 1;
  auto plan = q35::build_execution_plan(q35::qwen35_0_8b_shape(), warmup + steps, options);
  if (!check(plan.status(), "plan")) {
    return 1;
  }
  auto cache = q35::allocate_device_cache(ctx, plan.value());
  if (!check(cache.status(), "allocate_device_cache")) {
    return 1;
  }
  SyntheticModel sm(ctx);
  q35::ModelWeights w;
  if (!sm.build(plan.value(), w)) {
    return 1;
  }
  q35::DecodeScratch scratch;
  auto first =
    q35::greedy_decode(ctx, plan.value(), cache.value(), w, scratch, 11, 0, warmup, nullptr, order);
  if (!check(first.status(), "warmup decode")) {
    return 1;
  }
  const std::int32_t next = warmup > 0 ? first.value().back() : 11;
  const auto t0 = std::chrono::steady_clock::now();
  auto timed = q35::greedy_decode(ctx, plan.value(), cache.value(), w, scratch, next, warmup,
                                  steps, nullptr, order);
  const auto t1 = std::chrono::steady_clock::now();
  if (!check(timed.status(), "timed decode")) {
    return 1;
  }
  const double sec = std::chrono::duration<double>(t1 - t0).count();
  std::printf("decode tokens=%zu warmup=%zu ms_per_token=%.4f tok_s=%.1f weight_bytes=%llu "
              "weight_GB_s=%.1f\n",
              steps, warmup, 1e3 * sec / (double)steps, (double)steps / sec,
              (unsigned long long)sm.bytes(), (double)sm.bytes() * (double)steps / sec / 1e9);
  return 0;
}

int run_prefill(std::size_t prompt_tokens, std::size_t chunk_tokens, q35::OpOrder order) {
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  q35::RuntimeOptions options;
  options.prefill_chunk_tokens = chunk_tokens;
  auto plan = q35::build_execution_plan(q35::qwen35_0_8b_shape(), prompt_tokens, options);
  if (!check(plan.status(), "plan")) {
    return 1;
  }
  auto cache = q35::allocate_device_cache(ctx, plan.value());
  if (!check(cache.status(), "allocate_device_cache")) {
    return 1;
  }
  SyntheticModel sm(ctx);
  q35::ModelWeights w;
  if (!sm.build(plan.value(), w)) {
    return 1;
  }
  std::vector<std::int32_t> prompt(prompt_tokens);
  for (std::size_t i = 0; i < prompt_tokens; ++i) {
    prompt[i] = (std::int32_t)((7919u * i + 11u) % w.token_embd.rows);
  }
  q35::PrefillScratch ps;
  auto warm = q35::prefill_prompt(ctx, plan.value(), cache.value(), w, ps, prompt, nullptr, order);
  if (!check(warm.status(), "warmup prefill")) {
    return 1;
  }
  const auto t0 = std::chrono::steady_clock::now();
  auto timed = q35::prefill_prompt(ctx, plan.value(), cache.value(), w, ps, prompt, nullptr, order);
  const auto t1 = std::chrono::steady_clock::now();
  if (!check(timed.status(), "timed prefill")) {
    return 1;
  }
  const double sec = std::chrono::duration<double>(t1 - t0).count();
  std::printf("prefill prompt_tokens=%zu chunk_tokens=%zu chunks=%zu ms=%.3f tok_s=%.1f "
              "ms_per_chunk=%.3f\n",
              prompt_tokens, chunk_tokens, plan.value().prefill.chunk_count, 1e3 * sec,
              (double)prompt_tokens / sec, 1e3 * sec / (double)plan.value().prefill.chunk_count);
  return 0;
}

int run_prefix_store() {
  auto ctx_r = HipContext::create();
  if (!check(ctx_r.status(), "create")) {
    return 1;
  }
  const HipContext& ctx = ctx_r.value();
  constexpr std::size_t kBlock = 1024;
  constexpr int kBlocks = 8;
  q35::RuntimeOptions options;
  auto plan_r = q35::build_execution_plan(q35::qwen35_0_8b_shape(), kBlock * kBlocks, options);
  if (!check(plan_r.status(), "plan")) {
    return 1;
  }
  const q35::ExecutionPlan& plan = plan_r.value();
  auto cache_r = q35::allocate_device_cache(ctx, plan);
  auto hidden_b = ctx.make_buffer(kBlock * plan.hidden_size * sizeof(float));
  if (!check(cache_r.status(), "cache") || !check(hidden_b.status(), "hidden")) {
    return 1;
  }
  q35::DeviceCache& dc = cache_r.value();
  std::vector<std::int64_t> tokens(kBlock * kBlocks);
  for (std::size_t i = 0; i < tokens.size(); ++i) {
    tokens[i] = static_cast<std::int64_t>(i * 7919 % 151936);
  }
  q35::PrefixCacheStore store;
  store.configure(q35::prefix_layout_from_plan(plan, kBlock),
                  q35::PrefixCacheConfig{true, kBlock, kBlocks, 0});
  float sink = 0;
  auto sync = [&]() { return ctx.copy_from_buffer(hidden_b.value(), &sink, sizeof(sink)); };
  using clock = std::chrono::steady_clock;
  // The first commit allocates the store's arena; time the other blocks' commits.
  auto first = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, 0, kBlock);
  if (!check(first.status(), "commit") || !check(sync(), "sync")) {
    return 1;
  }
  auto t0 = clock::now();
  for (int i = 1; i < kBlocks; ++i) {
    auto c = store.commit_block(ctx, dc, plan, hidden_b.value(), tokens, i * kBlock, kBlock);
    if (!check(c.status(), "commit")) {
      return 1;
    }
  }
  if (!check(sync(), "sync")) {
    return 1;
  }
  const double commit_us =
    std::chrono::duration<double, std::micro>(clock::now() - t0).count() / (kBlocks - 1);
  const auto hit = store.lookup(tokens);
  constexpr int kRepeats = 20;
  t0 = clock::now();
  for (int i = 0; i < kRepeats; ++i) {
    if (!check(store.restore(ctx, dc, plan, hit.block_hashes), "restore")) {
      return 1;
    }
  }
  if (!check(sync(), "sync")) {
    return 1;
  }
  const double restore_us =
    std::chrono::duration<double, std::micro>(clock::now() - t0).count() / kRepeats;
  const double kv_block = 2.0 * plan.cache.full_attention_layers * kBlock * plan.cache.kv_dim *
                          plan.cache.kv_cache_element_bytes;
  const double recurrent =
    double(plan.cache.recurrent_r_cache_bytes + plan.cache.recurrent_s_cache_bytes);
  const double payload = kv_block + recurrent + plan.hidden_size * 4.0;
  const double restored = kBlocks * kv_block + recurrent;
  std::printf("prefix-store payload_bytes=%.0f hit_tokens=%zu commit_us=%.2f commit_GB_s=%.1f "
              "restore_us=%.2f restore_bytes=%.0f restore_GB_s=%.1f\n",
              payload, hit.hit_tokens, commit_us, payload / commit_us * 1e-3, restore_us,
              restored, restored / restore_us * 1e-3);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "";
  auto order_at = [&](int i) {
    return argc > i && std::string(argv[i]) == "reference" ? q35::OpOrder::reference
                                                           : q35::OpOrder::fused;
  };
  if (mode == "decode" && argc >= 4) {
    return run_decode(std::stoul(argv[2]), std::stoul(argv[3]), order_at(4));
  }
  if (mode == "prefill" && argc >= 4) {
    return run_prefill(std::stoul(argv[2]), std::stoul(argv[3]), order_at(4));
  }
  if (mode == "prefix-store") {
    return run_prefix_store();
  }
  std::printf("usage: qwen35_model_bench decode <warmup> <steps> [reference] | "
              "prefill <prompt_tokens> <chunk_tokens> [reference] | prefix-store\n");
  return 2;
}
