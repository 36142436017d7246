// C-ABI operator entry points: argument validation in the reference's order,
// then dispatch to the kernel launchers.  Messages follow the reference's
// wording with the "HIP" prefix in place of "MPS" (mps_backend.mm host
// dispatchers cited per function).
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "context_internal.hpp"

using namespace kraken;

namespace {

enum class FlashChoice { automatic, force_on, force_off };

// flash_attention_env_flag (mps_backend.mm:3716-3733): KRAKEN_QWEN35_FLASH_ATTENTION
// "1"/"true"/"on" forces flash, "0"/"false"/"off" disables it.
FlashChoice flash_env() {
  const char* v = std::getenv("KRAKEN_QWEN35_FLASH_ATTENTION");
  if (v == nullptr) {
    return FlashChoice::automatic;
  }
  if (!std::strcmp(v, "1") || !std::strcmp(v, "true") || !std::strcmp(v, "on")) {
    return FlashChoice::force_on;
  }
  if (!std::strcmp(v, "0") || !std::strcmp(v, "false") || !std::strcmp(v, "off")) {
    return FlashChoice::force_off;
  }
  return FlashChoice::automatic;
}

// attention_f32_batched[_f16_kv] host side (mps_backend.mm:10360-10617, 10619-10869).
int attention_entry(kraken_hip_context* ctx, const char* what, bool kv_f16,
                    const kraken_buffer& query, const kraken_buffer& key_cache,
                    const kraken_buffer& value_cache, const kraken_buffer* gate, size_t layer,
                    size_t start_position, size_t tokens, size_t capacity_tokens, size_t heads,
                    size_t kv_heads, size_t head_dim, const kraken_buffer& output,
                    bool no_alloc = false, bool query_f16 = false) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = std::string("HIP ") + what;
  if (tokens == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 || capacity_tokens == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (heads % kv_heads != 0) {
    return invalid(w + " heads must be divisible by kv_heads");
  }
  if (head_dim > 256u) {
    return invalid(w + " head_dim exceeds 256");
  }
  size_t key_count = 0;
  if (!checked_add(start_position, tokens, key_count) || key_count > capacity_tokens) {
    return invalid(w + " chunk exceeds KV cache capacity");
  }
  size_t attn_dim = 0, kv_dim = 0, query_values = 0, cache_layers = 0, cache_values = 0;
  if (!checked_mul(heads, head_dim, attn_dim) || !checked_mul(kv_heads, head_dim, kv_dim) ||
      !checked_mul(tokens, attn_dim, query_values) || layer == SIZE_MAX ||
      !checked_mul(layer + 1u, capacity_tokens, cache_layers) ||
      !checked_mul(cache_layers, kv_dim, cache_values)) {
    return invalid(w + " value count overflow");
  }
  const std::string nq = std::string(what) + " query";
  const std::string nk = std::string(what) + " key cache";
  const std::string nv = std::string(what) + " value cache";
  const std::string ng = std::string(what) + " gate";
  const std::string no = std::string(what) + " output";
  KRAKEN_TRY(validate_buffer(query, query_values, query_f16 ? sizeof(uint16_t) : sizeof(float),
                             nq.c_str()));
  const size_t elem = kv_f16 ? sizeof(uint16_t) : sizeof(float);
  KRAKEN_TRY(validate_buffer(key_cache, cache_values, elem, nk.c_str()));
  KRAKEN_TRY(validate_buffer(value_cache, cache_values, elem, nv.c_str()));
  if (gate != nullptr) {
    KRAKEN_TRY(validate_f32(*gate, query_values, ng.c_str()));
  }
  KRAKEN_TRY(validate_f32(output, query_values, no.c_str()));
  const std::string nl = std::string(what) + " layer";
  const std::string ns = std::string(what) + " start position";
  const std::string nt = std::string(what) + " tokens";
  const std::string nc = std::string(what) + " capacity";
  const std::string nh = std::string(what) + " heads";
  const std::string nkv = std::string(what) + " kv_heads";
  const std::string nd = std::string(what) + " head_dim";
  const std::string ngr = std::string(what) + " group";
  KRAKEN_TRY(check_u32(layer, nl.c_str()));
  KRAKEN_TRY(check_u32(start_position, ns.c_str()));
  KRAKEN_TRY(check_u32(tokens, nt.c_str()));
  KRAKEN_TRY(check_u32(capacity_tokens, nc.c_str()));
  KRAKEN_TRY(check_u32(heads, nh.c_str()));
  KRAKEN_TRY(check_u32(kv_heads, nkv.c_str()));
  KRAKEN_TRY(check_u32(head_dim, nd.c_str()));
  KRAKEN_TRY(check_u32(heads / kv_heads, ngr.c_str()));

  AttentionArgs a{};
  a.query = static_cast<const float*>(query.data);
  a.key_cache = key_cache.data;
  a.value_cache = value_cache.data;
  a.gate = gate != nullptr ? static_cast<const float*>(gate->data) : nullptr;
  a.output = static_cast<float*>(output.data);
  a.layer = (uint32_t)layer;
  a.start_position = (uint32_t)start_position;
  a.tokens = (uint32_t)tokens;
  a.capacity_tokens = (uint32_t)capacity_tokens;
  a.heads = (uint32_t)heads;
  a.kv_heads = (uint32_t)kv_heads;
  a.head_dim = (uint32_t)head_dim;
  a.kv_f16 = kv_f16;

  // Dispatch rule of the reference: flash for head_dim 256 and tokens >= 64,
  // overridable through the environment (mps_backend.mm:10715-10722).
  const FlashChoice choice = flash_env();
  const bool flash_ok = flash_prefill_supported(a);
  const bool use_flash = flash_ok && choice != FlashChoice::force_off &&
                         (choice == FlashChoice::force_on || tokens >= 64u);

  // An f16 query feeds the flash kernel as it is; the decode kernels read f32,
  // so that path widens it (exactly) into the workspace past the split partials.
  size_t need = use_flash ? attention_flash_workspace_bytes(a, ctx->cu_count)
                          : attention_decode_workspace_bytes(a, ctx->cu_count);
  size_t query_offset = 0;
  if (query_f16) {
    if (use_flash) {
      a.query = nullptr;
      a.query_f16 = query.data;
    } else {
      query_offset = (need + 255u) & ~size_t{255};
      need = query_offset + query_values * sizeof(float);
    }
  }
  if (no_alloc && need > kNoAllocScratchBytes) {
    return invalid(w + " needs " + std::to_string(need) +
                   " bytes of split partials; the allocation-free entry point has " +
                   std::to_string(kNoAllocScratchBytes));
  }
  KRAKEN_TRY(begin_launch(ctx));
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  if (no_alloc) {
    // Every split partial the kernels read is written earlier in the same
    // call, so the array needs no clearing between calls.
    workspace = ctx->no_alloc_scratch;
    workspace_bytes = kNoAllocScratchBytes;
  } else {
    KRAKEN_TRY(ensure_workspace(ctx, need));
    workspace = ctx->workspace;
    workspace_bytes = ctx->workspace_bytes;
  }
  if (query_f16 && !use_flash) {
    float* q32 = reinterpret_cast<float*>(static_cast<char*>(workspace) + query_offset);
    const hipError_t ec = launch_f16_to_f32(query.data, q32, query_values, ctx->stream);
    if (ec != hipSuccess) {
      return internal(w + " launch failed: " + hipGetErrorString(ec));
    }
    a.query = q32;
    workspace_bytes = query_offset;
  }
  const hipError_t e =
    use_flash ? launch_attention_flash(a, ctx->cu_count, workspace, workspace_bytes, ctx->stream)
              : launch_attention_decode(a, ctx->cu_count, workspace, workspace_bytes,
                                        ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

// gated_delta_net_f32_batched_in_place_at host side (mps_backend.mm:8517-8600).
int gdn_entry(kraken_hip_context* ctx, const char* what, const kraken_buffer& query,
              const kraken_buffer& key, const kraken_buffer& value, const kraken_buffer& gate,
              const kraken_buffer& beta, const kraken_buffer& state, size_t state_offset,
              size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim,
              const kraken_buffer& output, const kraken_buffer* dt_bias,
              const kraken_buffer* ssm_a, const kraken_buffer* z, const kraken_buffer* norm_w,
              float eps) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = std::string("HIP ") + what;
  if (tokens == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (value_heads % key_heads != 0) {
    return invalid(w + " value heads must repeat key heads");
  }
  if (head_dim > 256u) {
    return invalid(w + " head_dim exceeds 256");
  }
  size_t kvpt = 0, vvpt = 0, key_values = 0, value_values = 0, gate_values = 0, state_values = 0;
  if (!checked_mul(key_heads, head_dim, kvpt) || !checked_mul(value_heads, head_dim, vvpt) ||
      !checked_mul(tokens, kvpt, key_values) || !checked_mul(tokens, vvpt, value_values) ||
      !checked_mul(tokens, value_heads, gate_values) ||
      !checked_mul(vvpt, head_dim, state_values)) {
    return invalid(w + " value count overflow");
  }
  const std::string base(what);
  KRAKEN_TRY(validate_f32(query, key_values, (base + " query").c_str()));
  KRAKEN_TRY(validate_f32(key, key_values, (base + " key").c_str()));
  KRAKEN_TRY(validate_f32(value, value_values, (base + " value").c_str()));
  KRAKEN_TRY(validate_f32(gate, gate_values, (base + " gate").c_str()));
  KRAKEN_TRY(validate_f32(beta, gate_values, (base + " beta").c_str()));
  if (dt_bias != nullptr) {
    KRAKEN_TRY(validate_f32(*dt_bias, value_heads, (base + " dt bias").c_str()));
    KRAKEN_TRY(validate_f32(*ssm_a, value_heads, (base + " ssm a").c_str()));
    KRAKEN_TRY(validate_f32(*z, value_values, (base + " z").c_str()));
    KRAKEN_TRY(validate_f32(*norm_w, head_dim, (base + " norm weight").c_str()));
  }
  KRAKEN_TRY(validate_f32_region(state, state_offset, state_values, (base + " state").c_str()));
  KRAKEN_TRY(validate_f32(output, value_values, (base + " output").c_str()));
  KRAKEN_TRY(check_u32(tokens, (base + " tokens").c_str()));
  KRAKEN_TRY(check_u32(key_heads, (base + " key_heads").c_str()));
  KRAKEN_TRY(check_u32(value_heads, (base + " value_heads").c_str()));
  KRAKEN_TRY(check_u32(head_dim, (base + " head_dim").c_str()));
  KRAKEN_TRY(begin_launch(ctx));
  GdnArgs a{};
  a.query = static_cast<const float*>(query.data);
  a.key = static_cast<const float*>(key.data);
  a.value = static_cast<const float*>(value.data);
  a.gate = static_cast<const float*>(gate.data);
  a.beta = static_cast<const float*>(beta.data);
  a.state = static_cast<float*>(state.data) + state_offset;
  a.output = static_cast<float*>(output.data);
  a.tokens = (uint32_t)tokens;
  a.key_heads = (uint32_t)key_heads;
  a.value_heads = (uint32_t)value_heads;
  a.head_dim = (uint32_t)head_dim;
  if (dt_bias != nullptr) {
    a.dt_bias = static_cast<const float*>(dt_bias->data);
    a.ssm_a = static_cast<const float*>(ssm_a->data);
    a.z = static_cast<const float*>(z->data);
    a.norm_weight = static_cast<const float*>(norm_w->data);
    a.eps = eps;
  }
  KRAKEN_TRY(ensure_workspace(ctx, gdn_workspace_bytes(a)));
  const hipError_t e = launch_gated_delta_net(a, ctx->cu_count, ctx->workspace,
                                              ctx->workspace_bytes, ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

// qk_norm_f32_f32_batched / qwen35_norm_gated_f32_in_place host side
// (mps_backend.mm:8050-8210).
int rms_heads_entry(kraken_hip_context* ctx, const char* what, const kraken_buffer& values,
                    const kraken_buffer& weight, const kraken_buffer* gate, size_t tokens,
                    size_t heads, size_t head_dim, float eps) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = std::string("HIP ") + what;
  if (tokens == 0 || heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  const std::string base(what);
  KRAKEN_TRY(check_u32(tokens, (base + " tokens").c_str()));
  KRAKEN_TRY(check_u32(heads, (base + " heads").c_str()));
  KRAKEN_TRY(check_u32(head_dim, (base + " head_dim").c_str()));
  if (head_dim > 256u) {
    // One wave holds a whole head row (4 values per lane); the Metal kernel's
    // 256-thread groups have the same bound (mps_backend.mm:8090-8093).
    return invalid(w + " head_dim exceeds 256");
  }
  size_t head_values = 0, values_count = 0;
  if (!checked_mul(heads, head_dim, head_values) ||
      !checked_mul(tokens, head_values, values_count)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(values, values_count, (base + " values").c_str()));
  if (gate != nullptr) {
    KRAKEN_TRY(validate_f32(*gate, values_count, (base + " gate").c_str()));
  }
  KRAKEN_TRY(validate_f32(weight, head_dim, (base + " weight").c_str()));
  if (!fits_u32(tokens * heads)) {
    return invalid(w + " rows exceed uint32 range");
  }
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_rms_norm_heads(
    static_cast<float*>(values.data), static_cast<const float*>(weight.data),
    gate != nullptr ? static_cast<const float*>(gate->data) : nullptr, (uint32_t)tokens,
    (uint32_t)heads, (uint32_t)head_dim, eps, ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

// copy_f32_rows / copy_f32_rows_to_f16 / copy_f16_rows host side
// (mps_backend.mm:9694-9998).
int copy_rows_entry(kraken_hip_context* ctx, CopyKind kind, const char* what,
                    const kraken_buffer& source, const kraken_buffer& destination, size_t rows,
                    size_t row_size, size_t source_stride, size_t source_offset,
                    size_t destination_stride, size_t destination_offset) {
  KRAKEN_TRY(check_context(ctx));
  const std::string base(what);
  size_t source_end = 0, destination_end = 0;
  KRAKEN_TRY(strided_region_end(source_offset, rows, source_stride, row_size,
                                (base + " source").c_str(), source_end));
  KRAKEN_TRY(strided_region_end(destination_offset, rows, destination_stride, row_size,
                                (base + " destination").c_str(), destination_end));
  size_t total = 0;
  if (!checked_mul(rows, row_size, total)) {
    return invalid("HIP " + base + " value count overflow");
  }
  KRAKEN_TRY(check_u32(source_offset, (base + " source offset").c_str()));
  KRAKEN_TRY(check_u32(destination_offset, (base + " destination offset").c_str()));
  KRAKEN_TRY(check_u32(source_stride, (base + " source stride").c_str()));
  KRAKEN_TRY(check_u32(destination_stride, (base + " destination stride").c_str()));
  KRAKEN_TRY(check_u32(row_size, (base + " row size").c_str()));
  KRAKEN_TRY(check_u32(total, (base + " total").c_str()));
  const size_t src_elem = kind == CopyKind::f16 ? sizeof(uint16_t) : sizeof(float);
  const size_t dst_elem = kind == CopyKind::f32 ? sizeof(float) : sizeof(uint16_t);
  KRAKEN_TRY(validate_buffer(source, source_end, src_elem, (base + " source").c_str()));
  KRAKEN_TRY(
    validate_buffer(destination, destination_end, dst_elem, (base + " destination").c_str()));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e =
    launch_copy_rows(kind, source.data, destination.data, rows, row_size, source_stride,
                     source_offset, destination_stride, destination_offset, ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP " + base + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, ("HIP " + base + " command failed: ").c_str());
}

int unary_entry(kraken_hip_context* ctx, UnaryKind kind, const char* what,
                const kraken_buffer& values, size_t size) {
  KRAKEN_TRY(check_context(ctx));
  const std::string base(what);
  KRAKEN_TRY(check_u32(size, (base + " size").c_str()));
  KRAKEN_TRY(validate_f32(values, size, (base + " values").c_str()));
  KRAKEN_TRY(begin_launch(ctx));
  if (size == 0) {
    return KRAKEN_OK;
  }
  const hipError_t e = launch_unary(kind, static_cast<float*>(values.data), size, ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP " + base + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, ("HIP " + base + " command failed: ").c_str());
}

int binary_entry(kraken_hip_context* ctx, BinaryKind kind, const char* what,
                 const kraken_buffer& target, const kraken_buffer& rhs, size_t rows,
                 size_t row_size, bool rowwise, const char* target_name = nullptr,
                 const char* rhs_name = nullptr) {
  KRAKEN_TRY(check_context(ctx));
  const std::string base(what);
  size_t total = rows;
  if (rowwise) {
    if (rows == 0 || row_size == 0) {
      return invalid("HIP " + base + " dimensions must be positive");
    }
    if (!checked_mul(rows, row_size, total)) {
      return invalid("HIP " + base + " value count overflow");
    }
    KRAKEN_TRY(check_u32(row_size, (base + " row size").c_str()));
  }
  KRAKEN_TRY(check_u32(total, (base + " size").c_str()));
  const std::string tn = target_name != nullptr ? target_name : base + " target";
  const std::string rn = rhs_name != nullptr ? rhs_name : base + " rhs";
  KRAKEN_TRY(validate_f32(target, total, tn.c_str()));
  KRAKEN_TRY(validate_f32(rhs, rowwise ? row_size : total, rn.c_str()));
  KRAKEN_TRY(begin_launch(ctx));
  if (total == 0) {
    return KRAKEN_OK;
  }
  const hipError_t e = launch_binary(kind, static_cast<float*>(target.data),
                                     static_cast<const float*>(rhs.data), total,
                                     rowwise ? row_size : 1, ctx->stream);
  if (e != hipSuccess) {
    return internal("HIP " + base + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, ("HIP " + base + " command failed: ").c_str());
}

}  // namespace

extern "C" {

KRAKEN_API int kraken_hip_attention_f32_batched_f16_kv(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, size_t layer, size_t start_position, size_t tokens,
  size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim, kraken_buffer output) {
  return attention_entry(ctx, "F16 KV batched attention", true, query, key_cache, value_cache,
                         nullptr, layer, start_position, tokens, capacity_tokens, heads,
                         kv_heads, head_dim, output);
}

// No single counterpart in the reference: attention_f32_batched_f16_kv
// (mps_backend.mm:10619-10869) given a query that is f16 already.
KRAKEN_API int kraken_hip_attention_f16q_batched_f16_kv(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, size_t layer, size_t start_position, size_t tokens,
  size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim, kraken_buffer output) {
  return attention_entry(ctx, "F16 query F16 KV batched attention", true, query, key_cache,
                         value_cache, nullptr, layer, start_position, tokens, capacity_tokens,
                         heads, kv_heads, head_dim, output, /*no_alloc=*/false,
                         /*query_f16=*/true);
}

KRAKEN_API int kraken_hip_attention_f32_batched(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, size_t layer, size_t start_position, size_t tokens,
  size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim, kraken_buffer output) {
  return attention_entry(ctx, "batched attention", false, query, key_cache, value_cache,
                         nullptr, layer, start_position, tokens, capacity_tokens, heads,
                         kv_heads, head_dim, output);
}

KRAKEN_API int kraken_hip_attention_f32_batched_f16_kv_gated(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, kraken_buffer gate, size_t layer, size_t start_position,
  size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output) {
  return attention_entry(ctx, "gated F16 KV batched attention", true, query, key_cache,
                         value_cache, &gate, layer, start_position, tokens, capacity_tokens,
                         heads, kv_heads, head_dim, output);
}

// No counterpart in the reference: the gated F16-KV attention above with its
// split partials in the library's static per-device scratch array instead of
// context workspace, so it never allocates device memory.
KRAKEN_API int kraken_hip_attention_f32_batched_f16_kv_gated_no_alloc(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key_cache,
  kraken_buffer value_cache, kraken_buffer gate, size_t layer, size_t start_position,
  size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output) {
  return attention_entry(ctx, "gated F16 KV batched attention", true, query, key_cache,
                         value_cache, &gate, layer, start_position, tokens, capacity_tokens,
                         heads, kv_heads, head_dim, output, /*no_alloc=*/true);
}

KRAKEN_API int kraken_hip_gated_delta_net_f32_batched_in_place_at(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state, size_t state_offset,
  size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim, kraken_buffer output) {
  return gdn_entry(ctx, "batched gated delta net", query, key, value, gate, beta, state,
                   state_offset, tokens, key_heads, value_heads, head_dim, output, nullptr,
                   nullptr, nullptr, nullptr, 0.0f);
}

KRAKEN_API int kraken_hip_gated_delta_net_f32_batched_in_place(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state, size_t tokens, size_t key_heads,
  size_t value_heads, size_t head_dim, kraken_buffer output) {
  return gdn_entry(ctx, "batched gated delta net", query, key, value, gate, beta, state, 0,
                   tokens, key_heads, value_heads, head_dim, output, nullptr, nullptr, nullptr,
                   nullptr, 0.0f);
}

KRAKEN_API int kraken_hip_gated_delta_net_f32_in_place_at(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state, size_t state_offset,
  size_t key_heads, size_t value_heads, size_t head_dim, kraken_buffer output) {
  return gdn_entry(ctx, "gated delta net", query, key, value, gate, beta, state, state_offset,
                   1, key_heads, value_heads, head_dim, output, nullptr, nullptr, nullptr,
                   nullptr, 0.0f);
}

KRAKEN_API int kraken_hip_qwen35_gdn_gated_f32(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer alpha, kraken_buffer beta_raw, kraken_buffer dt_bias, kraken_buffer ssm_a,
  kraken_buffer z, kraken_buffer norm_weight, kraken_buffer state, size_t state_offset,
  size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim, float eps,
  kraken_buffer output) {
  return gdn_entry(ctx, "Qwen3.5 gated GDN", query, key, value, alpha, beta_raw, state,
                   state_offset, tokens, key_heads, value_heads, head_dim, output, &dt_bias,
                   &ssm_a, &z, &norm_weight, eps);
}

// ssm_conv_f32 host side (mps_backend.mm:8703-8799).
KRAKEN_API int kraken_hip_ssm_conv_f32(kraken_hip_context* ctx, kraken_buffer input,
                                       kraken_buffer kernel, size_t conv_kernel, size_t channels,
                                       size_t tokens, size_t sequences, kraken_buffer output) {
  KRAKEN_TRY(check_context(ctx));
  if (conv_kernel == 0 || channels == 0 || tokens == 0 || sequences == 0) {
    return invalid("HIP SSM conv dimensions must be positive");
  }
  size_t span = 0;
  if (!checked_add(conv_kernel - 1u, tokens, span)) {
    return invalid("HIP SSM conv input span overflow");
  }
  size_t input_values = 0, kernel_values = 0, output_values = 0;
  if (!checked_mul(span, channels, input_values) ||
      !checked_mul(input_values, sequences, input_values) ||
      !checked_mul(conv_kernel, channels, kernel_values) ||
      !checked_mul(channels, tokens, output_values) ||
      !checked_mul(output_values, sequences, output_values)) {
    return invalid("HIP SSM conv value count overflow");
  }
  KRAKEN_TRY(validate_f32(input, input_values, "SSM conv input"));
  KRAKEN_TRY(validate_f32(kernel, kernel_values, "SSM conv kernel"));
  KRAKEN_TRY(validate_f32(output, output_values, "SSM conv output"));
  KRAKEN_TRY(check_u32(conv_kernel, "SSM conv kernel"));
  KRAKEN_TRY(check_u32(span, "SSM conv input span"));
  KRAKEN_TRY(check_u32(channels, "SSM conv channels"));
  KRAKEN_TRY(check_u32(tokens, "SSM conv tokens"));
  KRAKEN_TRY(check_u32(sequences, "SSM conv sequences"));
  KRAKEN_TRY(check_u32(output_values, "SSM conv output values"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_ssm_conv(
    static_cast<const float*>(input.data), static_cast<const float*>(kernel.data),
    static_cast<float*>(output.data), (uint32_t)conv_kernel, (uint32_t)channels,
    (uint32_t)tokens, (uint32_t)sequences, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP SSM conv launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP SSM conv command failed: ");
}

// build_ssm_conv_state_f32 host side (mps_backend.mm:8801-8912).
KRAKEN_API int kraken_hip_build_ssm_conv_state_f32(kraken_hip_context* ctx, kraken_buffer state,
                                                   size_t state_offset, kraken_buffer input,
                                                   size_t conv_kernel, size_t channels,
                                                   size_t tokens, kraken_buffer conv_input) {
  KRAKEN_TRY(check_context(ctx));
  if (conv_kernel < 2 || channels == 0 || tokens == 0) {
    return invalid("HIP SSM conv-state dimensions are invalid");
  }
  size_t span = 0;
  if (!checked_add(conv_kernel - 1u, tokens, span)) {
    return invalid("HIP SSM conv-state input span overflow");
  }
  size_t state_values = 0, input_values = 0, conv_input_values = 0;
  if (!checked_mul(conv_kernel - 1u, channels, state_values) ||
      !checked_mul(tokens, channels, input_values) ||
      !checked_mul(span, channels, conv_input_values)) {
    return invalid("HIP SSM conv-state value count overflow");
  }
  KRAKEN_TRY(validate_f32_region(state, state_offset, state_values, "SSM conv-state state"));
  KRAKEN_TRY(validate_f32(input, input_values, "SSM conv-state input"));
  KRAKEN_TRY(validate_f32(conv_input, conv_input_values, "SSM conv-state conv input"));
  KRAKEN_TRY(check_u32(conv_kernel, "SSM conv-state kernel"));
  KRAKEN_TRY(check_u32(channels, "SSM conv-state channels"));
  KRAKEN_TRY(check_u32(tokens, "SSM conv-state tokens"));
  KRAKEN_TRY(check_u32(span, "SSM conv-state input span"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_build_ssm_conv_state(
    static_cast<float*>(state.data) + state_offset, static_cast<const float*>(input.data),
    static_cast<float*>(conv_input.data), (uint32_t)conv_kernel, (uint32_t)channels,
    (uint32_t)tokens, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP SSM conv-state launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP SSM conv-state command failed: ");
}

// ssm_conv1_f32_stateful_at host side (mps_backend.mm:8914-8990).
KRAKEN_API int kraken_hip_ssm_conv1_f32_stateful_at(kraken_hip_context* ctx, kraken_buffer state,
                                                    size_t state_offset, kraken_buffer input,
                                                    kraken_buffer kernel, size_t conv_kernel,
                                                    size_t channels, kraken_buffer output) {
  KRAKEN_TRY(check_context(ctx));
  if (conv_kernel < 2 || channels == 0) {
    return invalid("HIP stateful SSM conv dimensions are invalid");
  }
  size_t state_values = 0, kernel_values = 0;
  if (!checked_mul(conv_kernel - 1u, channels, state_values) ||
      !checked_mul(conv_kernel, channels, kernel_values)) {
    return invalid("HIP stateful SSM conv value count overflow");
  }
  KRAKEN_TRY(validate_f32_region(state, state_offset, state_values, "stateful SSM conv state"));
  KRAKEN_TRY(validate_f32(input, channels, "stateful SSM conv input"));
  KRAKEN_TRY(validate_f32(kernel, kernel_values, "stateful SSM conv kernel"));
  KRAKEN_TRY(validate_f32(output, channels, "stateful SSM conv output"));
  KRAKEN_TRY(check_u32(conv_kernel, "stateful SSM conv kernel"));
  KRAKEN_TRY(check_u32(channels, "stateful SSM conv channels"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_ssm_conv1_stateful(
    static_cast<float*>(state.data) + state_offset, static_cast<const float*>(input.data),
    static_cast<const float*>(kernel.data), static_cast<float*>(output.data),
    (uint32_t)conv_kernel, (uint32_t)channels, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP stateful SSM conv launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP stateful SSM conv command failed: ");
}

// Fused prologue of run_qwen35_linear_layer_chunk (qwen35_runtime.cpp:2746-2796).
KRAKEN_API int kraken_hip_qwen35_conv_split_l2_f32(
  kraken_hip_context* ctx, kraken_buffer qkv, kraken_buffer conv_state, size_t state_offset,
  kraken_buffer conv_kernel_weights, size_t conv_kernel, size_t tokens, size_t key_heads,
  size_t value_heads, size_t head_dim, float eps, kraken_buffer query, kraken_buffer key,
  kraken_buffer value) {
  KRAKEN_TRY(check_context(ctx));
  if (tokens == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid("HIP Qwen3.5 conv split dimensions must be positive");
  }
  if (conv_kernel < 2 || conv_kernel > 8) {
    return invalid("HIP Qwen3.5 conv split conv_kernel must be in [2, 8]");
  }
  if (head_dim > 256u) {
    return invalid("HIP Qwen3.5 conv split head_dim exceeds 256");
  }
  size_t key_dim = 0, value_dim = 0, channels = 0, qkv_values = 0, key_values = 0,
         value_values = 0, state_values = 0, kernel_values = 0;
  if (!checked_mul(key_heads, head_dim, key_dim) ||
      !checked_mul(value_heads, head_dim, value_dim) ||
      !checked_add(2u * key_dim, value_dim, channels) ||
      !checked_mul(tokens, channels, qkv_values) || !checked_mul(tokens, key_dim, key_values) ||
      !checked_mul(tokens, value_dim, value_values) ||
      !checked_mul(conv_kernel - 1u, channels, state_values) ||
      !checked_mul(conv_kernel, channels, kernel_values)) {
    return invalid("HIP Qwen3.5 conv split value count overflow");
  }
  KRAKEN_TRY(validate_f32(qkv, qkv_values, "Qwen3.5 conv split qkv"));
  KRAKEN_TRY(validate_f32_region(conv_state, state_offset, state_values,
                                 "Qwen3.5 conv split conv state"));
  KRAKEN_TRY(validate_f32(conv_kernel_weights, kernel_values, "Qwen3.5 conv split kernel"));
  KRAKEN_TRY(validate_f32(query, key_values, "Qwen3.5 conv split query"));
  KRAKEN_TRY(validate_f32(key, key_values, "Qwen3.5 conv split key"));
  KRAKEN_TRY(validate_f32(value, value_values, "Qwen3.5 conv split value"));
  KRAKEN_TRY(check_u32(tokens, "Qwen3.5 conv split tokens"));
  KRAKEN_TRY(check_u32(channels, "Qwen3.5 conv split channels"));
  KRAKEN_TRY(check_u32(qkv_values, "Qwen3.5 conv split qkv values"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_conv_split_l2(
    static_cast<const float*>(qkv.data), static_cast<float*>(conv_state.data) + state_offset,
    static_cast<const float*>(conv_kernel_weights.data), (uint32_t)conv_kernel,
    (uint32_t)tokens, (uint32_t)key_heads, (uint32_t)value_heads, (uint32_t)head_dim, eps,
    static_cast<float*>(query.data), static_cast<float*>(key.data),
    static_cast<float*>(value.data), ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP Qwen3.5 conv split launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP Qwen3.5 conv split command failed: ");
}

// split_qkv_l2_norm_f32_qwen35 host side (mps_backend.mm:8261-8377).
KRAKEN_API int kraken_hip_split_qkv_l2_norm_f32_qwen35(
  kraken_hip_context* ctx, kraken_buffer source, kraken_buffer query, kraken_buffer key,
  kraken_buffer value, size_t tokens, size_t key_heads, size_t value_heads, size_t head_dim,
  float eps) {
  KRAKEN_TRY(check_context(ctx));
  if (tokens == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid("HIP Qwen3.5 split qkv dimensions must be positive");
  }
  size_t key_dim = 0, value_dim = 0, doubled = 0, channels = 0;
  if (!checked_mul(key_heads, head_dim, key_dim) ||
      !checked_mul(value_heads, head_dim, value_dim) || !checked_mul(2u, key_dim, doubled) ||
      !checked_add(doubled, value_dim, channels)) {
    return invalid("HIP Qwen3.5 split qkv channel count overflow");
  }
  size_t source_values = 0, key_values = 0, value_values = 0;
  if (!checked_mul(tokens, channels, source_values) ||
      !checked_mul(tokens, key_dim, key_values) ||
      !checked_mul(tokens, value_dim, value_values)) {
    return invalid("HIP Qwen3.5 split qkv value count overflow");
  }
  KRAKEN_TRY(check_u32(tokens, "Qwen3.5 split qkv tokens"));
  KRAKEN_TRY(check_u32(key_heads, "Qwen3.5 split qkv key heads"));
  KRAKEN_TRY(check_u32(value_heads, "Qwen3.5 split qkv value heads"));
  KRAKEN_TRY(check_u32(head_dim, "Qwen3.5 split qkv head dim"));
  KRAKEN_TRY(check_u32(channels, "Qwen3.5 split qkv conv channels"));
  KRAKEN_TRY(validate_f32(source, source_values, "Qwen3.5 split qkv source"));
  KRAKEN_TRY(validate_f32(query, key_values, "Qwen3.5 split qkv query"));
  KRAKEN_TRY(validate_f32(key, key_values, "Qwen3.5 split qkv key"));
  KRAKEN_TRY(validate_f32(value, value_values, "Qwen3.5 split qkv value"));
  if (!fits_u32(tokens * (2u * key_heads + value_heads))) {
    return invalid("HIP Qwen3.5 split qkv row count exceeds uint32 range");
  }
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_split_qkv_l2(
    static_cast<const float*>(source.data), static_cast<float*>(query.data),
    static_cast<float*>(key.data), static_cast<float*>(value.data), (uint32_t)tokens,
    (uint32_t)key_heads, (uint32_t)value_heads, (uint32_t)head_dim, eps, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP Qwen3.5 split qkv launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP Qwen3.5 split qkv command failed: ");
}

// l2_norm_f32_in_place host side (mps_backend.mm:8211-8259).
KRAKEN_API int kraken_hip_l2_norm_f32_in_place(kraken_hip_context* ctx, kraken_buffer values,
                                               size_t rows, size_t row_size, float eps) {
  KRAKEN_TRY(check_context(ctx));
  if (rows == 0 || row_size == 0) {
    return invalid("HIP l2 norm dimensions must be positive");
  }
  KRAKEN_TRY(check_u32(rows, "l2 norm rows"));
  KRAKEN_TRY(check_u32(row_size, "l2 norm row size"));
  size_t total = 0;
  if (!checked_mul(rows, row_size, total)) {
    return invalid("HIP l2 norm value count overflow");
  }
  KRAKEN_TRY(validate_f32(values, total, "l2 norm values"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_l2_norm(static_cast<float*>(values.data), (uint32_t)rows,
                                      (uint32_t)row_size, eps, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP l2 norm launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP l2 norm command failed: ");
}

KRAKEN_API int kraken_hip_qk_norm_f32_f32_batched(kraken_hip_context* ctx, kraken_buffer values,
                                                  kraken_buffer weight, size_t tokens,
                                                  size_t heads, size_t head_dim, float eps) {
  return rms_heads_entry(ctx, "batched qk norm", values, weight, nullptr, tokens, heads,
                         head_dim, eps);
}

KRAKEN_API int kraken_hip_qwen35_norm_gated_f32_in_place(kraken_hip_context* ctx,
                                                         kraken_buffer values,
                                                         kraken_buffer weight,
                                                         kraken_buffer gate, size_t tokens,
                                                         size_t heads, size_t head_dim,
                                                         float eps) {
  return rms_heads_entry(ctx, "Qwen3.5 norm-gated", values, weight, &gate, tokens, heads,
                         head_dim, eps);
}

// prepare_qwen35_gdn_gate_beta_f32 host side (mps_backend.mm:9468-9540).
KRAKEN_API int kraken_hip_prepare_qwen35_gdn_gate_beta_f32(
  kraken_hip_context* ctx, kraken_buffer gate, kraken_buffer beta, kraken_buffer gate_bias,
  kraken_buffer gate_scale, size_t rows, size_t row_size) {
  KRAKEN_TRY(check_context(ctx));
  if (rows == 0 || row_size == 0) {
    return invalid("HIP Qwen3.5 GDN gate dimensions must be positive");
  }
  size_t total = 0;
  if (!checked_mul(rows, row_size, total)) {
    return invalid("HIP Qwen3.5 GDN gate value count overflow");
  }
  KRAKEN_TRY(check_u32(row_size, "Qwen3.5 GDN gate row size"));
  KRAKEN_TRY(check_u32(total, "Qwen3.5 GDN gate total"));
  KRAKEN_TRY(validate_f32(gate, total, "Qwen3.5 GDN gate"));
  KRAKEN_TRY(validate_f32(beta, total, "Qwen3.5 GDN beta"));
  KRAKEN_TRY(validate_f32(gate_bias, row_size, "Qwen3.5 GDN gate bias"));
  KRAKEN_TRY(validate_f32(gate_scale, row_size, "Qwen3.5 GDN gate scale"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_prepare_gate_beta(
    static_cast<float*>(gate.data), static_cast<float*>(beta.data),
    static_cast<const float*>(gate_bias.data), static_cast<const float*>(gate_scale.data),
    (uint32_t)rows, (uint32_t)row_size, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP Qwen3.5 GDN gate launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP Qwen3.5 GDN gate command failed: ");
}

// mrope_f32_in_place host side (mps_backend.mm:9057-9163).
KRAKEN_API int kraken_hip_mrope_f32_in_place(kraken_hip_context* ctx, kraken_buffer values,
                                             kraken_buffer positions, size_t tokens, size_t heads,
                                             size_t head_dim, size_t n_dims, size_t section_0,
                                             size_t section_1, size_t section_2,
                                             size_t section_3, float theta) {
  KRAKEN_TRY(check_context(ctx));
  if (tokens == 0 || heads == 0 || head_dim == 0 || n_dims == 0 || n_dims > head_dim ||
      n_dims % 2u != 0) {
    return invalid("HIP MRoPE dimensions are invalid");
  }
  size_t sections = 0;
  if (!checked_add(section_0, section_1, sections) ||
      !checked_add(sections, section_2, sections) ||
      !checked_add(sections, section_3, sections)) {
    return invalid("HIP MRoPE sections overflow");
  }
  if (sections == 0) {
    return invalid("HIP MRoPE sections must not all be zero");
  }
  size_t value_count = 0;
  if (!checked_mul(tokens, heads, value_count) ||
      !checked_mul(value_count, head_dim, value_count)) {
    return invalid("HIP MRoPE value count overflow");
  }
  KRAKEN_TRY(validate_f32(values, value_count, "MRoPE values"));
  size_t position_count = 0;
  if (!checked_mul(tokens, 4u, position_count)) {
    return invalid("HIP MRoPE position count overflow");
  }
  if (positions.data == nullptr || positions.byte_size < position_count * sizeof(int32_t)) {
    return invalid("HIP MRoPE position buffer is too small");
  }
  KRAKEN_TRY(check_u32(tokens, "MRoPE tokens"));
  KRAKEN_TRY(check_u32(heads, "MRoPE heads"));
  KRAKEN_TRY(check_u32(head_dim, "MRoPE head dim"));
  KRAKEN_TRY(check_u32(n_dims, "MRoPE n_dims"));
  KRAKEN_TRY(check_u32(section_0, "MRoPE section 0"));
  KRAKEN_TRY(check_u32(section_1, "MRoPE section 1"));
  KRAKEN_TRY(check_u32(section_2, "MRoPE section 2"));
  KRAKEN_TRY(check_u32(section_3, "MRoPE section 3"));
  KRAKEN_TRY(check_u32(sections, "MRoPE sections"));
  size_t pair_count = 0;
  if (!checked_mul(tokens, heads, pair_count) || !checked_mul(pair_count, n_dims / 2u, pair_count)) {
    return invalid("HIP MRoPE pair count overflow");
  }
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_mrope(
    static_cast<float*>(values.data), static_cast<const int32_t*>(positions.data),
    (uint32_t)tokens, (uint32_t)heads, (uint32_t)head_dim, (uint32_t)n_dims,
    (uint32_t)section_0, (uint32_t)section_1, (uint32_t)section_2, (uint32_t)section_3, theta,
    ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP MRoPE launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP MRoPE command failed: ");
}

namespace {

// Validation and argument block of the attention prologue entries.
int prologue_args(kraken_hip_context* ctx, const kraken_buffer& q_gate, const kraken_buffer& key,
                  const kraken_buffer& value, const kraken_buffer& q_norm,
                  const kraken_buffer& k_norm, const kraken_buffer& positions,
                  size_t mrope_start_position, const kraken_buffer& key_cache,
                  const kraken_buffer& value_cache, size_t layer, size_t start_position,
                  size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads,
                  size_t head_dim, size_t n_dims, size_t section_0, size_t section_1,
                  size_t section_2, size_t section_3, float theta, float eps,
                  const kraken_buffer& query_out, const kraken_buffer& gate_out,
                  PrologueArgs& a) {
  KRAKEN_TRY(check_context(ctx));
  if (tokens == 0 || heads == 0 || kv_heads == 0 || head_dim == 0 || capacity_tokens == 0) {
    return invalid("HIP attention prologue dimensions must be positive");
  }
  if (heads % kv_heads != 0) {
    return invalid("HIP attention prologue heads must be divisible by kv_heads");
  }
  if (head_dim > 256u) {
    return invalid("HIP attention prologue head_dim exceeds 256");
  }
  if (n_dims == 0 || n_dims > head_dim || n_dims % 2u != 0) {
    return invalid("HIP MRoPE dimensions are invalid");
  }
  size_t sections = 0;
  if (!checked_add(section_0, section_1, sections) ||
      !checked_add(sections, section_2, sections) ||
      !checked_add(sections, section_3, sections)) {
    return invalid("HIP MRoPE sections overflow");
  }
  if (sections == 0) {
    return invalid("HIP MRoPE sections must not all be zero");
  }
  size_t key_count = 0;
  if (!checked_add(start_position, tokens, key_count) || key_count > capacity_tokens) {
    return invalid("HIP attention prologue chunk exceeds KV cache capacity");
  }
  size_t attn_dim = 0, kv_dim = 0, query_values = 0, kv_values = 0, cache_rows = 0,
         cache_values = 0, joint_values = 0, position_count = 0;
  if (!checked_mul(heads, head_dim, attn_dim) || !checked_mul(kv_heads, head_dim, kv_dim) ||
      !checked_mul(tokens, attn_dim, query_values) ||
      !checked_mul(query_values, 2u, joint_values) ||
      !checked_mul(tokens, kv_dim, kv_values) || layer == SIZE_MAX ||
      !checked_mul(layer + 1u, capacity_tokens, cache_rows) ||
      !checked_mul(cache_rows, kv_dim, cache_values) || !checked_mul(tokens, 4u, position_count)) {
    return invalid("HIP attention prologue value count overflow");
  }
  KRAKEN_TRY(validate_f32(q_gate, joint_values, "attention prologue q_gate"));
  KRAKEN_TRY(validate_f32(key, kv_values, "attention prologue key"));
  KRAKEN_TRY(validate_f32(value, kv_values, "attention prologue value"));
  KRAKEN_TRY(validate_f32(q_norm, head_dim, "attention prologue q_norm"));
  KRAKEN_TRY(validate_f32(k_norm, head_dim, "attention prologue k_norm"));
  if (positions.data != nullptr) {
    KRAKEN_TRY(validate_i32(positions, position_count, "attention prologue positions"));
  }
  KRAKEN_TRY(validate_f16(key_cache, cache_values, "attention prologue key cache"));
  KRAKEN_TRY(validate_f16(value_cache, cache_values, "attention prologue value cache"));
  KRAKEN_TRY(validate_f32(query_out, query_values, "attention prologue query output"));
  KRAKEN_TRY(validate_f32(gate_out, query_values, "attention prologue gate output"));
  KRAKEN_TRY(check_u32(tokens, "attention prologue tokens"));
  KRAKEN_TRY(check_u32(heads + 2u * kv_heads, "attention prologue head slots"));
  KRAKEN_TRY(check_u32(n_dims, "MRoPE n_dims"));
  KRAKEN_TRY(check_u32(sections, "MRoPE sections"));
  if (positions.data == nullptr) {
    size_t last = 0;
    if (!checked_add(mrope_start_position, tokens - 1u, last) ||
        last > (size_t)std::numeric_limits<int32_t>::max()) {
      return invalid("Qwen3.5 batched MRoPE position exceeds int32 range");
    }
  }

  a = PrologueArgs{};
  a.q_gate = static_cast<const float*>(q_gate.data);
  a.key = static_cast<const float*>(key.data);
  a.value = static_cast<const float*>(value.data);
  a.q_norm = static_cast<const float*>(q_norm.data);
  a.k_norm = static_cast<const float*>(k_norm.data);
  a.positions = static_cast<const int32_t*>(positions.data);
  a.mrope_start = (uint32_t)mrope_start_position;
  a.key_cache = static_cast<_Float16*>(key_cache.data);
  a.value_cache = static_cast<_Float16*>(value_cache.data);
  a.cache_offset = (layer * capacity_tokens + start_position) * kv_dim;
  a.query_out = static_cast<float*>(query_out.data);
  a.gate_out = static_cast<float*>(gate_out.data);
  a.tokens = (uint32_t)tokens;
  a.heads = (uint32_t)heads;
  a.kv_heads = (uint32_t)kv_heads;
  a.head_dim = (uint32_t)head_dim;
  a.n_dims = (uint32_t)n_dims;
  a.s0 = (uint32_t)section_0;
  a.s1 = (uint32_t)section_1;
  a.s2 = (uint32_t)section_2;
  a.s3 = (uint32_t)section_3;
  a.theta = theta;
  a.eps = eps;
  return KRAKEN_OK;
}

}  // namespace

KRAKEN_API int kraken_hip_qwen35_attention_prologue_f16_kv(
  kraken_hip_context* ctx, kraken_buffer q_gate, kraken_buffer key, kraken_buffer value,
  kraken_buffer q_norm, kraken_buffer k_norm, kraken_buffer positions,
  size_t mrope_start_position, kraken_buffer key_cache, kraken_buffer value_cache, size_t layer,
  size_t start_position, size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads,
  size_t head_dim, size_t n_dims, size_t section_0, size_t section_1, size_t section_2,
  size_t section_3, float theta, float eps, kraken_buffer query_out, kraken_buffer gate_out) {
  PrologueArgs a{};
  KRAKEN_TRY(prologue_args(ctx, q_gate, key, value, q_norm, k_norm, positions,
                           mrope_start_position, key_cache, value_cache, layer, start_position,
                           tokens, capacity_tokens, heads, kv_heads, head_dim, n_dims, section_0,
                           section_1, section_2, section_3, theta, eps, query_out, gate_out, a));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_attention_prologue(a, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP attention prologue launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP attention prologue command failed: ");
}

// The prologue followed by the gated attention over the cache it appends to
// (the fused op order of run_full_attention_chunk, qwen35_runtime.cpp:
// 3229-3355).  One decode token within the single-split range runs as one
// launch; anything else as the prologue entry then the gated F16 KV attention
// entry, through query_out and gate_out.
KRAKEN_API int kraken_hip_qwen35_attention_prologue_gated_f16_kv(
  kraken_hip_context* ctx, kraken_buffer q_gate, kraken_buffer key, kraken_buffer value,
  kraken_buffer q_norm, kraken_buffer k_norm, kraken_buffer positions,
  size_t mrope_start_position, kraken_buffer key_cache, kraken_buffer value_cache, size_t layer,
  size_t start_position, size_t tokens, size_t capacity_tokens, size_t heads, size_t kv_heads,
  size_t head_dim, size_t n_dims, size_t section_0, size_t section_1, size_t section_2,
  size_t section_3, float theta, float eps, kraken_buffer query_out, kraken_buffer gate_out,
  kraken_buffer output) {
  PrologueArgs a{};
  KRAKEN_TRY(prologue_args(ctx, q_gate, key, value, q_norm, k_norm, positions,
                           mrope_start_position, key_cache, value_cache, layer, start_position,
                           tokens, capacity_tokens, heads, kv_heads, head_dim, n_dims, section_0,
                           section_1, section_2, section_3, theta, eps, query_out, gate_out, a));
  KRAKEN_TRY(validate_f32(output, tokens * heads * head_dim, "attention prologue output"));
  KRAKEN_TRY(check_u32(layer, "attention prologue layer"));
  KRAKEN_TRY(check_u32(capacity_tokens, "attention prologue capacity"));
  const char* order = std::getenv("KRAKEN_QWEN35_ATTENTION_PROLOGUE");
  if (order == nullptr || std::strcmp(order, "two_launch") != 0) {
    KRAKEN_TRY(begin_launch(ctx));
    const hipError_t e = launch_attention_prologue_decode(
      a, (uint32_t)layer, (uint32_t)start_position, (uint32_t)capacity_tokens,
      static_cast<float*>(output.data), ctx->stream);
    if (e == hipSuccess) {
      return finish_launch(ctx, "HIP attention prologue decode command failed: ");
    }
    if (e != hipErrorNotSupported) {
      return internal(std::string("HIP attention prologue decode launch failed: ") +
                      hipGetErrorString(e));
    }
  }
  KRAKEN_TRY(kraken_hip_qwen35_attention_prologue_f16_kv(
    ctx, q_gate, key, value, q_norm, k_norm, positions, mrope_start_position, key_cache,
    value_cache, layer, start_position, tokens, capacity_tokens, heads, kv_heads, head_dim,
    n_dims, section_0, section_1, section_2, section_3, theta, eps, query_out, gate_out));
  return attention_entry(ctx, "gated F16 KV batched attention", true, query_out, key_cache,
                         value_cache, &gate_out, layer, start_position, tokens, capacity_tokens,
                         heads, kv_heads, head_dim, output);
}

KRAKEN_API int kraken_hip_copy_f32_rows_to_f16(kraken_hip_context* ctx, kraken_buffer source,
                                               kraken_buffer destination, size_t rows,
                                               size_t row_size, size_t source_stride,
                                               size_t source_offset, size_t destination_stride,
                                               size_t destination_offset) {
  return copy_rows_entry(ctx, CopyKind::f32_to_f16, "copy rows to f16", source, destination,
                         rows, row_size, source_stride, source_offset, destination_stride,
                         destination_offset);
}

KRAKEN_API int kraken_hip_copy_f32_rows(kraken_hip_context* ctx, kraken_buffer source,
                                        kraken_buffer destination, size_t rows, size_t row_size,
                                        size_t source_stride, size_t source_offset,
                                        size_t destination_stride, size_t destination_offset) {
  return copy_rows_entry(ctx, CopyKind::f32, "copy rows", source, destination, rows, row_size,
                         source_stride, source_offset, destination_stride, destination_offset);
}

KRAKEN_API int kraken_hip_copy_f16_rows(kraken_hip_context* ctx, kraken_buffer source,
                                        kraken_buffer destination, size_t rows, size_t row_size,
                                        size_t source_stride, size_t source_offset,
                                        size_t destination_stride, size_t destination_offset) {
  return copy_rows_entry(ctx, CopyKind::f16, "copy f16 rows", source, destination, rows,
                         row_size, source_stride, source_offset, destination_stride,
                         destination_offset);
}

KRAKEN_API int kraken_hip_sigmoid_f32_in_place(kraken_hip_context* ctx, kraken_buffer values,
                                               size_t size) {
  return unary_entry(ctx, UnaryKind::sigmoid, "sigmoid", values, size);
}

KRAKEN_API int kraken_hip_softplus_f32_in_place(kraken_hip_context* ctx, kraken_buffer values,
                                                size_t size) {
  return unary_entry(ctx, UnaryKind::softplus, "softplus", values, size);
}

KRAKEN_API int kraken_hip_silu_f32_in_place(kraken_hip_context* ctx, kraken_buffer values,
                                            size_t size) {
  return unary_entry(ctx, UnaryKind::silu, "silu", values, size);
}

KRAKEN_API int kraken_hip_mul_f32_in_place(kraken_hip_context* ctx, kraken_buffer target,
                                           kraken_buffer rhs, size_t size) {
  return binary_entry(ctx, BinaryKind::mul, "mul", target, rhs, size, 0, false);
}

KRAKEN_API int kraken_hip_add_f32_in_place(kraken_hip_context* ctx, kraken_buffer target,
                                           kraken_buffer delta, size_t size) {
  return binary_entry(ctx, BinaryKind::add, "add", target, delta, size, 0, false, "add target",
                      "add delta");
}

KRAKEN_API int kraken_hip_silu_mul_f32_in_place(kraken_hip_context* ctx, kraken_buffer gate,
                                                kraken_buffer up, size_t size) {
  return binary_entry(ctx, BinaryKind::silu_mul, "silu mul", gate, up, size, 0, false,
                      "silu gate", "silu up");
}

// rms_norm_f32_f32_batched host side (mps_backend.mm:7865-7935): output[t] =
// input[t] * rsqrt(mean(input[t]^2) + eps) * weight, one row of `size` per token.
KRAKEN_API int kraken_hip_rms_norm_f32_f32_batched(kraken_hip_context* ctx, kraken_buffer input,
                                                   kraken_buffer weight, size_t tokens,
                                                   size_t size, float eps,
                                                   kraken_buffer output) {
  KRAKEN_TRY(check_context(ctx));
  if (tokens == 0 || size == 0) {
    return invalid("HIP batched rms norm dimensions must be positive");
  }
  KRAKEN_TRY(check_u32(tokens, "batched rms norm tokens"));
  KRAKEN_TRY(check_u32(size, "batched rms norm size"));
  size_t values = 0;
  if (!checked_mul(tokens, size, values)) {
    return invalid("HIP batched rms norm value count overflow");
  }
  KRAKEN_TRY(validate_f32(input, values, "batched rms norm input"));
  KRAKEN_TRY(validate_f32(output, values, "batched rms norm output"));
  KRAKEN_TRY(validate_f32(weight, size, "batched rms norm weight"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_rms_norm_rows(
    static_cast<const float*>(input.data), static_cast<const float*>(weight.data),
    static_cast<float*>(output.data), (uint32_t)tokens, (uint32_t)size, eps, ctx->stream);
  if (e != hipSuccess) {
    return internal(std::string("HIP batched rms norm launch failed: ") + hipGetErrorString(e));
  }
  return finish_launch(ctx, "HIP batched rms norm command failed: ");
}

KRAKEN_API int kraken_hip_add_f32_row_in_place(kraken_hip_context* ctx, kraken_buffer target,
                                               kraken_buffer row, size_t rows, size_t row_size) {
  return binary_entry(ctx, BinaryKind::add_row, "add row", target, row, rows, row_size, true);
}

KRAKEN_API int kraken_hip_mul_f32_row_in_place(kraken_hip_context* ctx, kraken_buffer target,
                                               kraken_buffer row, size_t rows, size_t row_size) {
  return binary_entry(ctx, BinaryKind::mul_row, "mul row", target, row, rows, row_size, true);
}

}  // extern "C"

namespace {

// ---------------------------------------------------------------------------
// Ragged multi-sequence decode (no counterpart in the reference, which serves
// one sequence per context; README.md:540).  Each sequence contributes one
// token.  Per-sequence tables live in device memory (u64 element offsets into
// caller-owned pools, u32 positions) so a captured step can be replayed while
// the caller advances them on the device.  Offsets are not readable on the
// host: kernels bound every access to the pool instead (an offset outside it
// skips that sequence's state, or reads zeros from the KV pool).

// Elements of a pool buffer of `elem` bytes per element; invalid when the byte
// size is not a whole number of elements.
int pool_elems_of(const kraken_buffer& pool, size_t elem, size_t at_least, const std::string& w,
                  const char* name, uint64_t& elems) {
  KRAKEN_TRY(validate_buffer(pool, at_least, elem, name));
  if (pool.byte_size % elem != 0) {
    return invalid(w + " " + name + " size is not a whole number of elements");
  }
  elems = pool.byte_size / elem;
  return KRAKEN_OK;
}

int ragged_attention_entry(kraken_hip_context* ctx, const kraken_buffer& query,
                           const kraken_buffer& key_pool, const kraken_buffer& value_pool,
                           const kraken_buffer* gate, const kraken_buffer& seq_kv_offsets,
                           const kraken_buffer& seq_positions, size_t sequences,
                           size_t max_position, size_t heads, size_t kv_heads, size_t head_dim,
                           const kraken_buffer& output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = "HIP ragged attention";
  if (sequences == 0 || heads == 0 || kv_heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (heads % kv_heads != 0) {
    return invalid(w + " heads must be divisible by kv_heads");
  }
  const size_t group = heads / kv_heads;
  if ((head_dim != 64 && head_dim != 128 && head_dim != 256) ||
      (group != 1 && group != 2 && group != 4 && group != 8)) {
    return invalid(w + " supports head_dim 64/128/256 and 1/2/4/8 query heads per kv head");
  }
  if (((uintptr_t)query.data | (uintptr_t)key_pool.data | (uintptr_t)value_pool.data |
       (uintptr_t)output.data) & 15u) {
    return invalid(w + " buffers must be 16-byte aligned");
  }
  size_t attn_dim = 0, kv_dim = 0, query_values = 0, one_sequence = 0;
  if (max_position >= 0xffffffffu || !checked_mul(heads, head_dim, attn_dim) ||
      !checked_mul(kv_heads, head_dim, kv_dim) ||
      !checked_mul(sequences, attn_dim, query_values) ||
      !checked_mul(max_position + 1u, kv_dim, one_sequence)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(query, query_values, "ragged attention query"));
  uint64_t pool_elems = 0, value_elems = 0;
  KRAKEN_TRY(pool_elems_of(key_pool, sizeof(uint16_t), kv_dim, w, "ragged attention key pool",
                           pool_elems));
  KRAKEN_TRY(pool_elems_of(value_pool, sizeof(uint16_t), kv_dim, w,
                           "ragged attention value pool", value_elems));
  if (value_elems != pool_elems) {
    return invalid(w + " key and value pools differ in size");
  }
  if (gate != nullptr) {
    KRAKEN_TRY(validate_f32(*gate, query_values, "ragged attention gate"));
  }
  KRAKEN_TRY(validate_buffer(seq_kv_offsets, sequences, sizeof(uint64_t),
                             "ragged attention kv offsets"));
  KRAKEN_TRY(validate_buffer(seq_positions, sequences, sizeof(uint32_t),
                             "ragged attention positions"));
  KRAKEN_TRY(validate_f32(output, query_values, "ragged attention output"));
  KRAKEN_TRY(check_u32(sequences, "ragged attention sequences"));
  KRAKEN_TRY(check_u32(heads, "ragged attention heads"));
  KRAKEN_TRY(check_u32(kv_heads, "ragged attention kv_heads"));

  AttentionArgs a{};
  a.query = static_cast<const float*>(query.data);
  a.key_cache = key_pool.data;
  a.value_cache = value_pool.data;
  a.gate = gate != nullptr ? static_cast<const float*>(gate->data) : nullptr;
  a.output = static_cast<float*>(output.data);
  a.tokens = (uint32_t)sequences;
  a.heads = (uint32_t)heads;
  a.kv_heads = (uint32_t)kv_heads;
  a.head_dim = (uint32_t)head_dim;
  a.kv_f16 = true;
  a.seq_kv_offsets = static_cast<const uint64_t*>(seq_kv_offsets.data);
  a.seq_positions = static_cast<const uint32_t*>(seq_positions.data);
  a.pool_elems = pool_elems;
  a.max_position = (uint32_t)max_position;
  KRAKEN_TRY(begin_launch(ctx));
  KRAKEN_TRY(ensure_workspace(ctx, attention_decode_workspace_bytes(a, ctx->cu_count)));
  const hipError_t e = launch_attention_decode(a, ctx->cu_count, ctx->workspace,
                                               ctx->workspace_bytes, ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

}  // namespace

extern "C" {

KRAKEN_API int kraken_hip_attention_f32_ragged_f16_kv(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key_pool, kraken_buffer value_pool,
  kraken_buffer gate, kraken_buffer seq_kv_offsets, kraken_buffer seq_positions,
  size_t sequences, size_t max_position, size_t heads, size_t kv_heads, size_t head_dim,
  kraken_buffer output) {
  return ragged_attention_entry(ctx, query, key_pool, value_pool,
                                gate.data != nullptr ? &gate : nullptr, seq_kv_offsets,
                                seq_positions, sequences, max_position, heads, kv_heads,
                                head_dim, output);
}

KRAKEN_API int kraken_hip_append_kv_ragged_f16(kraken_hip_context* ctx, kraken_buffer key_rows,
                                               kraken_buffer value_rows, kraken_buffer key_pool,
                                               kraken_buffer value_pool,
                                               kraken_buffer seq_kv_offsets,
                                               kraken_buffer seq_positions, size_t sequences,
                                               size_t row_size) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = "HIP ragged KV append";
  if (sequences == 0 || row_size == 0) {
    return invalid(w + " dimensions must be positive");
  }
  size_t values = 0;
  if (!checked_mul(sequences, row_size, values)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(key_rows, values, "ragged KV append key rows"));
  KRAKEN_TRY(validate_f32(value_rows, values, "ragged KV append value rows"));
  uint64_t pool_elems = 0, value_elems = 0;
  KRAKEN_TRY(pool_elems_of(key_pool, sizeof(uint16_t), row_size, w, "ragged KV append key pool",
                           pool_elems));
  KRAKEN_TRY(pool_elems_of(value_pool, sizeof(uint16_t), row_size, w,
                           "ragged KV append value pool", value_elems));
  if (value_elems != pool_elems) {
    return invalid(w + " key and value pools differ in size");
  }
  KRAKEN_TRY(validate_buffer(seq_kv_offsets, sequences, sizeof(uint64_t),
                             "ragged KV append kv offsets"));
  KRAKEN_TRY(validate_buffer(seq_positions, sequences, sizeof(uint32_t),
                             "ragged KV append positions"));
  KRAKEN_TRY(check_u32(sequences, "ragged KV append sequences"));
  KRAKEN_TRY(check_u32(row_size, "ragged KV append row size"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_append_kv_ragged(
    static_cast<const float*>(key_rows.data), static_cast<const float*>(value_rows.data),
    key_pool.data, value_pool.data, static_cast<const uint64_t*>(seq_kv_offsets.data),
    static_cast<const uint32_t*>(seq_positions.data), pool_elems, (uint32_t)sequences,
    (uint32_t)row_size, ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

KRAKEN_API int kraken_hip_gated_delta_net_f32_ragged_decode(
  kraken_hip_context* ctx, kraken_buffer query, kraken_buffer key, kraken_buffer value,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer state_pool,
  kraken_buffer seq_state_offsets, size_t sequences, size_t key_heads, size_t value_heads,
  size_t head_dim, kraken_buffer output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = "HIP ragged gated delta net";
  if (sequences == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (value_heads % key_heads != 0) {
    return invalid(w + " value heads must repeat key heads");
  }
  if (head_dim > 256u) {
    return invalid(w + " head_dim exceeds 256");
  }
  size_t kvpt = 0, vvpt = 0, key_values = 0, value_values = 0, gate_values = 0,
         state_values = 0;
  if (!checked_mul(key_heads, head_dim, kvpt) || !checked_mul(value_heads, head_dim, vvpt) ||
      !checked_mul(sequences, kvpt, key_values) || !checked_mul(sequences, vvpt, value_values) ||
      !checked_mul(sequences, value_heads, gate_values) ||
      !checked_mul(vvpt, head_dim, state_values)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(query, key_values, "ragged gated delta net query"));
  KRAKEN_TRY(validate_f32(key, key_values, "ragged gated delta net key"));
  KRAKEN_TRY(validate_f32(value, value_values, "ragged gated delta net value"));
  KRAKEN_TRY(validate_f32(gate, gate_values, "ragged gated delta net gate"));
  KRAKEN_TRY(validate_f32(beta, gate_values, "ragged gated delta net beta"));
  uint64_t pool_elems = 0;
  KRAKEN_TRY(pool_elems_of(state_pool, sizeof(float), state_values, w,
                           "ragged gated delta net state pool", pool_elems));
  KRAKEN_TRY(validate_buffer(seq_state_offsets, sequences, sizeof(uint64_t),
                             "ragged gated delta net state offsets"));
  KRAKEN_TRY(validate_f32(output, value_values, "ragged gated delta net output"));
  KRAKEN_TRY(check_u32(sequences, "ragged gated delta net sequences"));
  KRAKEN_TRY(check_u32(key_heads, "ragged gated delta net key_heads"));
  KRAKEN_TRY(check_u32(value_heads, "ragged gated delta net value_heads"));
  KRAKEN_TRY(begin_launch(ctx));
  GdnArgs a{};
  a.query = static_cast<const float*>(query.data);
  a.key = static_cast<const float*>(key.data);
  a.value = static_cast<const float*>(value.data);
  a.gate = static_cast<const float*>(gate.data);
  a.beta = static_cast<const float*>(beta.data);
  a.state = static_cast<float*>(state_pool.data);
  a.output = static_cast<float*>(output.data);
  a.tokens = (uint32_t)sequences;
  a.key_heads = (uint32_t)key_heads;
  a.value_heads = (uint32_t)value_heads;
  a.head_dim = (uint32_t)head_dim;
  a.seq_state_offsets = static_cast<const uint64_t*>(seq_state_offsets.data);
  a.pool_elems = pool_elems;
  const hipError_t e = launch_gated_delta_net(a, ctx->cu_count, nullptr, 0, ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

KRAKEN_API int kraken_hip_qwen35_conv_split_l2_ragged_decode_f32(
  kraken_hip_context* ctx, kraken_buffer qkv, kraken_buffer conv_pool,
  kraken_buffer seq_conv_offsets, kraken_buffer conv_kernel_weights, size_t conv_kernel,
  size_t sequences, size_t key_heads, size_t value_heads, size_t head_dim, float eps,
  kraken_buffer query, kraken_buffer key, kraken_buffer value) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = "HIP ragged Qwen3.5 conv split";
  if (sequences == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (conv_kernel < 2 || conv_kernel > 8) {
    return invalid(w + " conv_kernel must be in [2, 8]");
  }
  if (head_dim > 256u) {
    return invalid(w + " head_dim exceeds 256");
  }
  size_t key_dim = 0, value_dim = 0, channels = 0, qkv_values = 0, key_values = 0,
         value_values = 0, state_values = 0, kernel_values = 0;
  if (!checked_mul(key_heads, head_dim, key_dim) ||
      !checked_mul(value_heads, head_dim, value_dim) ||
      !checked_add(2u * key_dim, value_dim, channels) ||
      !checked_mul(sequences, channels, qkv_values) ||
      !checked_mul(sequences, key_dim, key_values) ||
      !checked_mul(sequences, value_dim, value_values) ||
      !checked_mul(conv_kernel - 1u, channels, state_values) ||
      !checked_mul(conv_kernel, channels, kernel_values)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(qkv, qkv_values, "ragged Qwen3.5 conv split qkv"));
  uint64_t pool_elems = 0;
  KRAKEN_TRY(pool_elems_of(conv_pool, sizeof(float), state_values, w,
                           "ragged Qwen3.5 conv split conv pool", pool_elems));
  KRAKEN_TRY(validate_buffer(seq_conv_offsets, sequences, sizeof(uint64_t),
                             "ragged Qwen3.5 conv split conv offsets"));
  KRAKEN_TRY(validate_f32(conv_kernel_weights, kernel_values, "ragged Qwen3.5 conv split kernel"));
  KRAKEN_TRY(validate_f32(query, key_values, "ragged Qwen3.5 conv split query"));
  KRAKEN_TRY(validate_f32(key, key_values, "ragged Qwen3.5 conv split key"));
  KRAKEN_TRY(validate_f32(value, value_values, "ragged Qwen3.5 conv split value"));
  KRAKEN_TRY(check_u32(sequences, "ragged Qwen3.5 conv split sequences"));
  KRAKEN_TRY(check_u32(channels, "ragged Qwen3.5 conv split channels"));
  KRAKEN_TRY(begin_launch(ctx));
  const hipError_t e = launch_conv_split_l2_ragged(
    static_cast<const float*>(qkv.data), static_cast<float*>(conv_pool.data),
    static_cast<const uint64_t*>(seq_conv_offsets.data), pool_elems,
    static_cast<const float*>(conv_kernel_weights.data), (uint32_t)conv_kernel,
    (uint32_t)sequences, (uint32_t)key_heads, (uint32_t)value_heads, (uint32_t)head_dim, eps,
    static_cast<float*>(query.data), static_cast<float*>(key.data),
    static_cast<float*>(value.data), ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

// No counterpart in the reference: the gated delta rule of
// kraken_hip_qwen35_gdn_layer_ragged_decode_f32 for a qkv whose conv and SiLU
// are already applied (by kraken_hip_kquant_matvec_multi_conv_f32), output
// y * scale and gate_output the norm-gated epilogue's norm_weight * silu(z),
// each head over 8 or 16 workgroups.
KRAKEN_API int kraken_hip_qwen35_gdn_state_ragged_decode_f32(
  kraken_hip_context* ctx, kraken_buffer qkv, kraken_buffer gate, kraken_buffer beta,
  kraken_buffer dt_bias, kraken_buffer ssm_a, kraken_buffer z, kraken_buffer norm_weight,
  kraken_buffer state_pool, kraken_buffer seq_state_offsets, size_t sequences,
  size_t key_heads, size_t value_heads, size_t head_dim, float eps, kraken_buffer output,
  kraken_buffer gate_output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = "HIP ragged Qwen3.5 GDN state";
  if (sequences == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (head_dim != 128 || key_heads != value_heads) {
    return invalid(w + " needs head_dim 128 and key_heads == value_heads");
  }
  if ((dt_bias.data == nullptr) != (ssm_a.data == nullptr)) {
    return invalid(w + " dt_bias and ssm_a must be given together");
  }
  size_t dim = 0, channels = 0, qkv_values = 0, value_values = 0, gate_values = 0,
         state_values = 0;
  if (!checked_mul(value_heads, head_dim, dim) || !checked_mul(3u, dim, channels) ||
      !checked_mul(sequences, channels, qkv_values) ||
      !checked_mul(sequences, dim, value_values) ||
      !checked_mul(sequences, value_heads, gate_values) ||
      !checked_mul(dim, head_dim, state_values)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(qkv, qkv_values, "ragged Qwen3.5 GDN state qkv"));
  KRAKEN_TRY(validate_f32(gate, gate_values, "ragged Qwen3.5 GDN state gate"));
  KRAKEN_TRY(validate_f32(beta, gate_values, "ragged Qwen3.5 GDN state beta"));
  if (dt_bias.data != nullptr) {
    KRAKEN_TRY(validate_f32(dt_bias, value_heads, "ragged Qwen3.5 GDN state dt_bias"));
    KRAKEN_TRY(validate_f32(ssm_a, value_heads, "ragged Qwen3.5 GDN state ssm_a"));
  }
  KRAKEN_TRY(validate_f32(z, value_values, "ragged Qwen3.5 GDN state z"));
  KRAKEN_TRY(validate_f32(norm_weight, head_dim, "ragged Qwen3.5 GDN state norm weight"));
  uint64_t state_elems = 0;
  KRAKEN_TRY(pool_elems_of(state_pool, sizeof(float), state_values, w,
                           "ragged Qwen3.5 GDN state pool", state_elems));
  KRAKEN_TRY(validate_buffer(seq_state_offsets, sequences, sizeof(uint64_t),
                             "ragged Qwen3.5 GDN state offsets"));
  KRAKEN_TRY(validate_f32(output, value_values, "ragged Qwen3.5 GDN state output"));
  KRAKEN_TRY(validate_f32(gate_output, value_values, "ragged Qwen3.5 GDN state gate output"));
  KRAKEN_TRY(check_u32(sequences, "ragged Qwen3.5 GDN state sequences"));
  KRAKEN_TRY(check_u32(value_heads, "ragged Qwen3.5 GDN state value_heads"));
  KRAKEN_TRY(begin_launch(ctx));
  GdnLayerArgs a{};
  a.qkv = static_cast<const float*>(qkv.data);
  a.gate = static_cast<const float*>(gate.data);
  a.beta = static_cast<const float*>(beta.data);
  a.dt_bias = static_cast<const float*>(dt_bias.data);
  a.ssm_a = static_cast<const float*>(ssm_a.data);
  a.z = static_cast<const float*>(z.data);
  a.norm_weight = static_cast<const float*>(norm_weight.data);
  a.state_pool = static_cast<float*>(state_pool.data);
  a.seq_state_offsets = static_cast<const uint64_t*>(seq_state_offsets.data);
  a.state_pool_elems = state_elems;
  a.output = static_cast<float*>(output.data);
  a.gate_factor = static_cast<float*>(gate_output.data);
  a.sequences = (uint32_t)sequences;
  a.heads = (uint32_t)value_heads;
  a.eps = eps;
  const hipError_t e = launch_gdn_state_ragged(a, ctx->stream);
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

// One decode step of the Qwen3.5 linear-attention core for many sequences: the
// ragged conv prologue, gated delta rule and norm-gated epilogue
// (qwen35_runtime.cpp:2740-3008 between the projections) in one kernel where
// the shape allows, else as the three-kernel chain.  No single MpsContext
// method corresponds.
KRAKEN_API int kraken_hip_qwen35_gdn_layer_ragged_decode_f32(
  kraken_hip_context* ctx, kraken_buffer qkv, kraken_buffer conv_pool,
  kraken_buffer seq_conv_offsets, kraken_buffer conv_kernel_weights, size_t conv_kernel,
  kraken_buffer gate, kraken_buffer beta, kraken_buffer dt_bias, kraken_buffer ssm_a,
  kraken_buffer z, kraken_buffer norm_weight, kraken_buffer state_pool,
  kraken_buffer seq_state_offsets, size_t sequences, size_t key_heads, size_t value_heads,
  size_t head_dim, float eps, kraken_buffer output) {
  KRAKEN_TRY(check_context(ctx));
  const std::string w = "HIP ragged Qwen3.5 GDN layer";
  if (sequences == 0 || key_heads == 0 || value_heads == 0 || head_dim == 0) {
    return invalid(w + " dimensions must be positive");
  }
  if (value_heads % key_heads != 0) {
    return invalid(w + " value heads must repeat key heads");
  }
  if (conv_kernel < 2 || conv_kernel > 8) {
    return invalid(w + " conv_kernel must be in [2, 8]");
  }
  if (head_dim > 256u) {
    return invalid(w + " head_dim exceeds 256");
  }
  if ((dt_bias.data == nullptr) != (ssm_a.data == nullptr)) {
    return invalid(w + " dt_bias and ssm_a must be given together");
  }
  size_t key_dim = 0, value_dim = 0, channels = 0, qkv_values = 0, key_values = 0,
         value_values = 0, conv_state_values = 0, kernel_values = 0, gate_values = 0,
         state_values = 0;
  if (!checked_mul(key_heads, head_dim, key_dim) ||
      !checked_mul(value_heads, head_dim, value_dim) ||
      !checked_add(2u * key_dim, value_dim, channels) ||
      !checked_mul(sequences, channels, qkv_values) ||
      !checked_mul(sequences, key_dim, key_values) ||
      !checked_mul(sequences, value_dim, value_values) ||
      !checked_mul(conv_kernel - 1u, channels, conv_state_values) ||
      !checked_mul(conv_kernel, channels, kernel_values) ||
      !checked_mul(sequences, value_heads, gate_values) ||
      !checked_mul(value_dim, head_dim, state_values)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(validate_f32(qkv, qkv_values, "ragged Qwen3.5 GDN layer qkv"));
  uint64_t conv_elems = 0, state_elems = 0;
  KRAKEN_TRY(pool_elems_of(conv_pool, sizeof(float), conv_state_values, w,
                           "ragged Qwen3.5 GDN layer conv pool", conv_elems));
  KRAKEN_TRY(validate_buffer(seq_conv_offsets, sequences, sizeof(uint64_t),
                             "ragged Qwen3.5 GDN layer conv offsets"));
  KRAKEN_TRY(validate_f32(conv_kernel_weights, kernel_values, "ragged Qwen3.5 GDN layer kernel"));
  KRAKEN_TRY(validate_f32(gate, gate_values, "ragged Qwen3.5 GDN layer gate"));
  KRAKEN_TRY(validate_f32(beta, gate_values, "ragged Qwen3.5 GDN layer beta"));
  if (dt_bias.data != nullptr) {
    KRAKEN_TRY(validate_f32(dt_bias, value_heads, "ragged Qwen3.5 GDN layer dt_bias"));
    KRAKEN_TRY(validate_f32(ssm_a, value_heads, "ragged Qwen3.5 GDN layer ssm_a"));
  }
  KRAKEN_TRY(validate_f32(z, value_values, "ragged Qwen3.5 GDN layer z"));
  KRAKEN_TRY(validate_f32(norm_weight, head_dim, "ragged Qwen3.5 GDN layer norm weight"));
  KRAKEN_TRY(pool_elems_of(state_pool, sizeof(float), state_values, w,
                           "ragged Qwen3.5 GDN layer state pool", state_elems));
  KRAKEN_TRY(validate_buffer(seq_state_offsets, sequences, sizeof(uint64_t),
                             "ragged Qwen3.5 GDN layer state offsets"));
  KRAKEN_TRY(validate_f32(output, value_values, "ragged Qwen3.5 GDN layer output"));
  KRAKEN_TRY(check_u32(sequences, "ragged Qwen3.5 GDN layer sequences"));
  KRAKEN_TRY(check_u32(channels, "ragged Qwen3.5 GDN layer channels"));
  KRAKEN_TRY(check_u32(value_heads, "ragged Qwen3.5 GDN layer value_heads"));

  const auto* dtb = static_cast<const float*>(dt_bias.data);
  const auto* ssa = static_cast<const float*>(ssm_a.data);
  if (gdn_layer_fused_supported((uint32_t)head_dim, (uint32_t)conv_kernel, (uint32_t)key_heads,
                                (uint32_t)value_heads)) {
    KRAKEN_TRY(begin_launch(ctx));
    GdnLayerArgs a{};
    a.qkv = static_cast<const float*>(qkv.data);
    a.conv_pool = static_cast<float*>(conv_pool.data);
    a.seq_conv_offsets = static_cast<const uint64_t*>(seq_conv_offsets.data);
    a.conv_pool_elems = conv_elems;
    a.conv_weights = static_cast<const float*>(conv_kernel_weights.data);
    a.gate = static_cast<const float*>(gate.data);
    a.beta = static_cast<const float*>(beta.data);
    a.dt_bias = dtb;
    a.ssm_a = ssa;
    a.z = static_cast<const float*>(z.data);
    a.norm_weight = static_cast<const float*>(norm_weight.data);
    a.state_pool = static_cast<float*>(state_pool.data);
    a.seq_state_offsets = static_cast<const uint64_t*>(seq_state_offsets.data);
    a.state_pool_elems = state_elems;
    a.output = static_cast<float*>(output.data);
    a.sequences = (uint32_t)sequences;
    a.heads = (uint32_t)value_heads;
    a.eps = eps;
    const hipError_t e = launch_gdn_layer_ragged(a, ctx->stream);
    if (e != hipSuccess) {
      return internal(w + " launch failed: " + hipGetErrorString(e));
    }
    return finish_launch(ctx, (w + " command failed: ").c_str());
  }

  // Three-kernel chain: q/k/v in the context workspace.
  size_t tmp_bytes = 0;
  if (!checked_mul(2u * key_values + value_values, sizeof(float), tmp_bytes)) {
    return invalid(w + " value count overflow");
  }
  KRAKEN_TRY(ensure_workspace(ctx, tmp_bytes));
  KRAKEN_TRY(begin_launch(ctx));
  float* qb = static_cast<float*>(ctx->workspace);
  float* kb = qb + key_values;
  float* vb = kb + key_values;
  hipError_t e = launch_conv_split_l2_ragged(
    static_cast<const float*>(qkv.data), static_cast<float*>(conv_pool.data),
    static_cast<const uint64_t*>(seq_conv_offsets.data), conv_elems,
    static_cast<const float*>(conv_kernel_weights.data), (uint32_t)conv_kernel,
    (uint32_t)sequences, (uint32_t)key_heads, (uint32_t)value_heads, (uint32_t)head_dim, eps,
    qb, kb, vb, ctx->stream);
  if (e == hipSuccess) {
    GdnArgs a{};
    a.query = qb;
    a.key = kb;
    a.value = vb;
    a.gate = static_cast<const float*>(gate.data);
    a.beta = static_cast<const float*>(beta.data);
    a.state = static_cast<float*>(state_pool.data);
    a.output = static_cast<float*>(output.data);
    a.tokens = (uint32_t)sequences;
    a.key_heads = (uint32_t)key_heads;
    a.value_heads = (uint32_t)value_heads;
    a.head_dim = (uint32_t)head_dim;
    a.dt_bias = dtb;
    a.ssm_a = ssa;
    a.seq_state_offsets = static_cast<const uint64_t*>(seq_state_offsets.data);
    a.pool_elems = state_elems;
    e = launch_gated_delta_net(a, ctx->cu_count, nullptr, 0, ctx->stream);
  }
  if (e == hipSuccess) {
    e = launch_rms_norm_heads(static_cast<float*>(output.data),
                              static_cast<const float*>(norm_weight.data),
                              static_cast<const float*>(z.data), (uint32_t)sequences,
                              (uint32_t)value_heads, (uint32_t)head_dim, eps, ctx->stream);
  }
  if (e != hipSuccess) {
    return internal(w + " launch failed: " + hipGetErrorString(e));
  }
  return finish_launch(ctx, (w + " command failed: ").c_str());
}

}  // extern "C"
