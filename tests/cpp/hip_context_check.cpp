// Drives the C++ mirror (include/kraken/hip_context.hpp) the way the reference
// runtime drives MpsContext.
//
//   hip_context_check cpu   no GPU needed: create() reports unavailable; a
//                           validation-only context returns invalid_argument
//                           for the reference's argument checks (in its order)
//                           and unavailable for accepted arguments.
//   hip_context_check gpu   on a GPU: decode attention through the wrapper
//                           against the closed form of smoke_test.cpp:1688-1725
//                           (zero query -> uniform mean of V over the causal
//                           prefix), gated variant (mean * sigmoid(G)), and a
//                           buffer round trip.
// Prints one line per check and exits non-zero on the first failure.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "kraken/hip_context.hpp"

using kraken::hip::HipBuffer;
using kraken::hip::HipContext;
using kraken::hip::Status;
using kraken::hip::StatusCode;

namespace {

int failures = 0;

void expect(bool ok, const std::string& what, const Status& s = Status::ok()) {
  std::printf("%s %s%s%s\n", ok ? "ok  " : "FAIL", what.c_str(), s.message().empty() ? "" : ": ",
              s.message().c_str());
  if (!ok) {
    ++failures;
  }
}

uint16_t to_half(float f) {
  // Round-to-nearest-even f32 -> f16 for finite values in the normal range.
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  int32_t exp = (int32_t)((x >> 23) & 0xFF) - 127 + 15;
  uint32_t mant = x & 0x7FFFFFu;
  if (exp <= 0) {
    return (uint16_t)sign;  // flush tiny values (inputs here are O(1))
  }
  uint32_t h = sign | ((uint32_t)exp << 10) | (mant >> 13);
  const uint32_t rest = mant & 0x1FFFu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) {
    ++h;
  }
  return (uint16_t)h;
}

float from_half(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1F;
  const uint32_t mant = h & 0x3FFu;
  uint32_t x = sign;
  if (exp != 0) {
    x |= ((exp - 15 + 127) << 23) | (mant << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

int run_cpu() {
  auto real = HipContext::create();
  expect(!real.is_ok() && real.status().code() == StatusCode::unavailable,
         "create() without a GPU reports unavailable", real.status());

  auto vo = HipContext::create_validation_only();
  expect(vo.is_ok(), "create_validation_only()", vo.status());
  if (!vo.is_ok()) {
    return 1;
  }
  const HipContext& ctx = vo.value();
  // Borrowed views with fake device addresses: validation reads only sizes.
  auto view = [](std::size_t bytes) {
    return HipBuffer::borrow(reinterpret_cast<void*>(uintptr_t{1} << 20), bytes);
  };
  const std::size_t heads = 8, kv_heads = 2, d = 256, cap = 33, tokens = 1, start = 31;
  HipBuffer q = view(4 * tokens * heads * d);
  HipBuffer kc = view(2 * cap * kv_heads * d);
  HipBuffer vc = view(2 * cap * kv_heads * d);
  HipBuffer out = view(4 * tokens * heads * d);

  Status s = ctx.attention_f32_batched_f16_kv(q, kc, vc, 0, start, tokens, cap, heads, kv_heads,
                                              d, out);
  expect(s.code() == StatusCode::unavailable, "valid decode arguments accepted", s);
  s = ctx.attention_f32_batched_f16_kv(q, kc, vc, 0, start, tokens, cap, heads, 3, d, out);
  expect(s.code() == StatusCode::invalid_argument, "heads % kv_heads != 0 rejected", s);
  s = ctx.attention_f32_batched_f16_kv(q, kc, vc, 0, 40, tokens, cap, heads, kv_heads, d, out);
  expect(s.code() == StatusCode::invalid_argument, "start + tokens > capacity rejected", s);
  s = ctx.attention_f32_batched_f16_kv(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, 512,
                                       out);
  expect(s.code() == StatusCode::invalid_argument, "head_dim > 256 rejected", s);
  HipBuffer small = view(16);
  s = ctx.attention_f32_batched_f16_kv(q, kc, vc, 0, start, tokens, cap, heads, kv_heads, d,
                                       small);
  expect(s.code() == StatusCode::invalid_argument, "short output buffer rejected", s);

  const std::size_t hk = 16, hv = 16, dd = 128, t = 4;
  HipBuffer gq = view(4 * t * hk * dd), gk = view(4 * t * hk * dd), gv = view(4 * t * hv * dd);
  HipBuffer gg = view(4 * t * hv), gb = view(4 * t * hv), st = view(4 * hv * dd * dd);
  HipBuffer go = view(4 * t * hv * dd);
  s = ctx.gated_delta_net_f32_batched_in_place_at(gq, gk, gv, gg, gb, st, 0, t, hk, hv, dd, go);
  expect(s.code() == StatusCode::unavailable, "valid GDN arguments accepted", s);
  s = ctx.gated_delta_net_f32_batched_in_place_at(gq, gk, gv, gg, gb, st, 1, t, hk, hv, dd, go);
  expect(s.code() == StatusCode::invalid_argument, "GDN state offset past the buffer rejected",
         s);

  // K-quant projections (Q5_K 6144 x 1024, the Qwen3.5 shape) and argmax.
  HipBuffer qw = view(6144 * 4 * 176), qx = view(4 * 1024 * 9), qy = view(4 * 6144 * 9);
  s = ctx.matmul_q5_k_f32_device(qw, 6144, 1024, 9, qx, qy);
  expect(s.code() == StatusCode::unavailable, "valid Q5_K matmul arguments accepted", s);
  s = ctx.matmul_q5_k_f32_device(qw, 6144, 1000, 9, qx, qy);
  expect(s.code() == StatusCode::invalid_argument &&
           s.message() == "HIP Q5_K matmul cols must be divisible by 256",
         "Q5_K matmul cols % 256 rejected", s);
  auto host = ctx.matvec_q4_k_f32(qw, 16, 1024, std::vector<float>(1000, 1.0f));
  expect(!host.is_ok() &&
           host.status().message() == "HIP Q4_K matvec input size does not match cols",
         "host-vector Q4_K matvec input size checked first", host.status());
  HipBuffer tok = view(4), prob = view(4);
  s = ctx.argmax_prob_f32_i32(qy, 0, tok, prob);
  expect(s.code() == StatusCode::invalid_argument &&
           s.message() == "HIP argmax probability size must be positive",
         "argmax_prob size 0 rejected", s);
  return failures == 0 ? 0 : 1;
}

int run_gpu() {
  auto created = HipContext::create();
  expect(created.is_ok(), "create()", created.status());
  if (!created.is_ok()) {
    return 1;
  }
  const HipContext& ctx = created.value();
  const std::size_t heads = 8, kv_heads = 2, d = 256, prior = 300, tokens = 1;
  const std::size_t cap = prior + tokens;
  std::mt19937_64 rng(1);
  std::normal_distribution<float> normal(0.0f, 1.0f);
  std::vector<uint16_t> kh(cap * kv_heads * d), vh(cap * kv_heads * d);
  for (auto& x : kh) x = to_half(normal(rng));
  for (auto& x : vh) x = to_half(normal(rng));
  std::vector<float> q(tokens * heads * d, 0.0f), gate(tokens * heads * d);
  for (auto& x : gate) x = normal(rng);

  auto make = [&](std::size_t bytes, const void* src) {
    auto r = ctx.make_buffer(bytes);
    expect(r.is_ok(), "make_buffer(" + std::to_string(bytes) + ")", r.status());
    HipBuffer b = std::move(r.value());
    if (src != nullptr) {
      const Status s = ctx.copy_to_buffer(b, src, bytes);
      expect(s.is_ok(), "copy_to_buffer", s);
    }
    return b;
  };
  HipBuffer qb = make(4 * q.size(), q.data());
  HipBuffer kb = make(2 * kh.size(), kh.data());
  HipBuffer vb = make(2 * vh.size(), vh.data());
  HipBuffer gb = make(4 * gate.size(), gate.data());
  HipBuffer ob = make(4 * q.size(), nullptr);
  HipBuffer og = make(4 * q.size(), nullptr);

  Status s = ctx.attention_f32_batched_f16_kv(qb, kb, vb, 0, prior, tokens, cap, heads,
                                              kv_heads, d, ob);
  expect(s.is_ok(), "attention_f32_batched_f16_kv", s);
  s = ctx.attention_f32_batched_f16_kv_gated(qb, kb, vb, gb, 0, prior, tokens, cap, heads,
                                             kv_heads, d, og);
  expect(s.is_ok(), "attention_f32_batched_f16_kv_gated", s);
  std::vector<float> out(q.size()), outg(q.size());
  s = ctx.copy_from_buffer(ob, out.data(), 4 * out.size());
  expect(s.is_ok(), "copy_from_buffer", s);
  s = ctx.copy_from_buffer(og, outg.data(), 4 * outg.size());
  expect(s.is_ok(), "copy_from_buffer (gated)", s);

  // Zero query: every key scores 0, so each head returns the mean of its KV
  // head's V rows over keys 0..prior (the new token included).
  double worst = 0.0, worst_g = 0.0;
  for (std::size_t h = 0; h < heads; ++h) {
    const std::size_t kvh = h / (heads / kv_heads);
    for (std::size_t c = 0; c < d; ++c) {
      double mean = 0.0;
      for (std::size_t j = 0; j <= prior; ++j) {
        mean += from_half(vh[(j * kv_heads + kvh) * d + c]);
      }
      mean /= (double)(prior + 1);
      const double sig = 1.0 / (1.0 + std::exp(-(double)gate[h * d + c]));
      worst = std::fmax(worst, std::fabs(out[h * d + c] - mean) / (1e-3 + 2e-3 * std::fabs(mean)));
      worst_g = std::fmax(worst_g, std::fabs(outg[h * d + c] - mean * sig) /
                                     (1e-3 + 2e-3 * std::fabs(mean * sig)));
    }
  }
  expect(worst <= 1.0, "zero-query decode equals the mean of V (2e-3 rel / 1e-3 abs)");
  expect(worst_g <= 1.0, "gated zero-query decode equals mean * sigmoid(G)");

  std::vector<float> back(q.size());
  s = ctx.copy_buffer_region(gb, ob, 0, 0, 4 * gate.size());
  expect(s.is_ok(), "copy_buffer_region", s);
  s = ctx.copy_from_buffer(ob, back.data(), 4 * back.size());
  expect(s.is_ok() && back == gate, "buffer round trip through copy_buffer_region", s);

  // The reference smoke test's Q4_K block (smoke_test.cpp:875-894): d = 1,
  // dmin = 0, all 6-bit scales 1, quants 0x21, so W x = 128 * 1 + 128 * 2 for
  // x = 1; then argmax_prob over {-1, 5, 2} (smoke_test.cpp:1622-1638).
  std::vector<uint8_t> block(144, 0);
  block[1] = 0x3C;
  for (int i = 4; i < 16; ++i) block[i] = 1;
  for (int i = 16; i < 144; ++i) block[i] = 0x21;
  HipBuffer wq = make(block.size(), block.data());
  auto mv = ctx.matvec_q4_k_f32(wq, 1, 256, std::vector<float>(256, 1.0f));
  expect(mv.is_ok() && mv.value().size() == 1 && std::fabs(mv.value()[0] - 384.0f) < 1e-5f,
         "host-vector Q4_K matvec known answer 384", mv.status());
  const float logits[3] = {-1.0f, 5.0f, 2.0f};
  HipBuffer lb = make(sizeof(logits), logits);
  HipBuffer tb = make(4, nullptr), pb = make(4, nullptr);
  s = ctx.argmax_prob_f32_i32(lb, 3, tb, pb);
  int32_t token = -1;
  float probability = 0.0f;
  expect(s.is_ok() && ctx.copy_from_buffer(tb, &token, 4).is_ok() &&
           ctx.copy_from_buffer(pb, &probability, 4).is_ok() && token == 1 &&
           std::fabs(probability - 0.950330f) < 1e-4f,
         "argmax_prob known answer (1, 0.950330)", s);
  return failures == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  const int rc = mode == "gpu" ? run_gpu() : run_cpu();
  std::printf("%s\n", rc == 0 ? "all checks passed" : "checks failed");
  return rc;
}
