// C++ mirror of the reference backend interface over the kraken HIP C ABI.
//
// kraken::hip::HipContext has the names, argument order and meaning, and the
// Status/Result error convention of the hot-path subset of
// toyllm::mps::MpsContext (include/toyllm/backends/mps/mps_backend.hpp:76-428,
// core/status.hpp:8-32), so a runtime written against that class can switch to
// this one by type alias (see the integration notes shipped with the library).
// Header-only: every method forwards to one extern "C" entry point of
// include/kraken_hip.h and turns its int status plus the thread-local message
// into a Status.  No exceptions cross the boundary.
//
// Ownership (mirrors MpsBuffer, mps_backend.hpp:26-47): a HipBuffer made by
// make_buffer owns one device allocation and frees it on destruction; a
// HipBuffer made by HipBuffer::borrow views caller-owned device memory (a torch
// tensor, a KV cache in another allocator) and frees nothing.  Ops never
// allocate caller-visible memory; *_at variants take element offsets.
//
// Threading: a context is used by one thread at a time; many contexts may live
// on different threads (each holds its own stream and workspace).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>
#include <utility>

#include "kraken_hip.h"

namespace kraken::hip {

enum class StatusCode { ok, invalid_argument, unavailable, internal_error };

class Status {
 public:
  Status() = default;
  Status(StatusCode code, std::string message) : code_(code), message_(std::move(message)) {}

  [[nodiscard]] static Status ok() { return Status(); }
  [[nodiscard]] static Status invalid_argument(std::string m) {
    return Status(StatusCode::invalid_argument, std::move(m));
  }
  [[nodiscard]] static Status unavailable(std::string m) {
    return Status(StatusCode::unavailable, std::move(m));
  }
  [[nodiscard]] static Status internal_error(std::string m) {
    return Status(StatusCode::internal_error, std::move(m));
  }

  [[nodiscard]] bool is_ok() const { return code_ == StatusCode::ok; }
  [[nodiscard]] StatusCode code() const { return code_; }
  [[nodiscard]] const std::string& message() const { return message_; }

  // C-ABI return code (0..3, same order as StatusCode) plus the calling
  // thread's last error message.
  [[nodiscard]] static Status from_code(int code) {
    switch (code) {
      case KRAKEN_OK:
        return ok();
      case KRAKEN_INVALID_ARGUMENT:
        return invalid_argument(kraken_hip_last_error());
      case KRAKEN_UNAVAILABLE:
        return unavailable(kraken_hip_last_error());
      default:
        return internal_error(kraken_hip_last_error());
    }
  }

 private:
  StatusCode code_{StatusCode::ok};
  std::string message_;
};

template <typename T>
class Result {
 public:
  Result(T value) : value_(std::move(value)), status_(Status::ok()) {}
  Result(Status status) : status_(std::move(status)) {}

  [[nodiscard]] bool is_ok() const { return status_.is_ok(); }
  [[nodiscard]] const Status& status() const { return status_; }
  [[nodiscard]] T& value() { return value_; }
  [[nodiscard]] const T& value() const { return value_; }

 private:
  T value_{};
  Status status_;
};

class HipContext;

// One device allocation (owned) or a view of caller-owned device memory.
class HipBuffer {
 public:
  HipBuffer() = default;
  ~HipBuffer() { reset(); }

  HipBuffer(const HipBuffer&) = delete;
  HipBuffer& operator=(const HipBuffer&) = delete;

  HipBuffer(HipBuffer&& other) noexcept
      : raw_(other.raw_), owner_(other.owner_) {
    other.raw_ = kraken_buffer{nullptr, 0};
    other.owner_ = nullptr;
  }
  HipBuffer& operator=(HipBuffer&& other) noexcept {
    if (this != &other) {
      reset();
      raw_ = other.raw_;
      owner_ = other.owner_;
      other.raw_ = kraken_buffer{nullptr, 0};
      other.owner_ = nullptr;
    }
    return *this;
  }

  // Non-owning view of `byte_size` bytes of device memory at `data`.
  [[nodiscard]] static HipBuffer borrow(void* data, std::size_t byte_size) {
    HipBuffer b;
    b.raw_ = kraken_buffer{data, byte_size};
    return b;
  }

  [[nodiscard]] bool valid() const { return raw_.data != nullptr; }
  [[nodiscard]] std::size_t byte_size() const { return raw_.byte_size; }
  [[nodiscard]] void* data() const { return raw_.data; }
  [[nodiscard]] kraken_buffer raw() const { return raw_; }

 private:
  friend class HipContext;

  void reset() {
    if (owner_ != nullptr && raw_.data != nullptr) {
      kraken_hip_free_buffer(owner_, &raw_);
    }
    raw_ = kraken_buffer{nullptr, 0};
    owner_ = nullptr;
  }

  kraken_buffer raw_{nullptr, 0};
  kraken_hip_context* owner_{nullptr};  // null for borrowed views
};

class HipContext {
 public:
  HipContext() = default;
  ~HipContext() {
    if (ctx_ != nullptr) {
      kraken_hip_context_destroy(ctx_);
    }
  }

  HipContext(const HipContext&) = delete;
  HipContext& operator=(const HipContext&) = delete;

  HipContext(HipContext&& other) noexcept : ctx_(other.ctx_) { other.ctx_ = nullptr; }
  HipContext& operator=(HipContext&& other) noexcept {
    if (this != &other) {
      if (ctx_ != nullptr) {
        kraken_hip_context_destroy(ctx_);
      }
      ctx_ = other.ctx_;
      other.ctx_ = nullptr;
    }
    return *this;
  }

  // mps_backend.hpp:87.  Unavailable (with the reason) when no GPU is usable.
  [[nodiscard]] static Result<HipContext> create() {
    kraken_hip_context* raw = nullptr;
    const Status s = Status::from_code(kraken_hip_context_create(&raw));
    if (!s.is_ok()) {
      return s;
    }
    return HipContext(raw);
  }

  // A context that runs every op's argument validation but launches nothing
  // (valid arguments return unavailable); usable without a GPU.
  [[nodiscard]] static Result<HipContext> create_validation_only() {
    kraken_hip_context* raw = nullptr;
    const Status s = Status::from_code(kraken_hip_context_create_validation_only(&raw));
    if (!s.is_ok()) {
      return s;
    }
    return HipContext(raw);
  }

  [[nodiscard]] bool valid() const { return ctx_ != nullptr; }
  [[nodiscard]] kraken_hip_context* raw() const { return ctx_; }

  // Enqueue on a caller's hipStream_t (nullptr restores the context's own).
  [[nodiscard]] Status set_stream(void* hip_stream) const {
    return Status::from_code(kraken_hip_context_set_stream(ctx_, hip_stream));
  }

  // mps_backend.hpp:92-94
  [[nodiscard]] Status begin_graph() const {
    return Status::from_code(kraken_hip_begin_graph(ctx_));
  }
  [[nodiscard]] Status commit_graph() const {
    return Status::from_code(kraken_hip_commit_graph(ctx_));
  }
  void abort_graph() const { kraken_hip_abort_graph(ctx_); }

  // mps_backend.hpp:96-114
  [[nodiscard]] Result<HipBuffer> make_buffer(std::size_t byte_size) const {
    HipBuffer b;
    const Status s = Status::from_code(kraken_hip_make_buffer(ctx_, byte_size, &b.raw_));
    if (!s.is_ok()) {
      return s;
    }
    b.owner_ = ctx_;
    return b;
  }
  [[nodiscard]] Status copy_to_buffer(HipBuffer& buffer, const void* data,
                                      std::size_t byte_size) const {
    return Status::from_code(kraken_hip_copy_to_buffer(ctx_, buffer.raw(), data, byte_size));
  }
  [[nodiscard]] Status copy_to_buffer_at(HipBuffer& buffer, std::size_t destination_offset,
                                         const void* data, std::size_t byte_size) const {
    return Status::from_code(
      kraken_hip_copy_to_buffer_at(ctx_, buffer.raw(), destination_offset, data, byte_size));
  }
  [[nodiscard]] Status copy_from_buffer(const HipBuffer& buffer, void* data,
                                        std::size_t byte_size) const {
    return Status::from_code(kraken_hip_copy_from_buffer(ctx_, buffer.raw(), data, byte_size));
  }
  [[nodiscard]] Status copy_from_buffer_at(const HipBuffer& buffer, std::size_t source_offset,
                                           void* data, std::size_t byte_size) const {
    return Status::from_code(
      kraken_hip_copy_from_buffer_at(ctx_, buffer.raw(), source_offset, data, byte_size));
  }
  [[nodiscard]] Status copy_buffer_region(const HipBuffer& source, HipBuffer& destination,
                                          std::size_t source_offset,
                                          std::size_t destination_offset,
                                          std::size_t byte_size) const {
    return Status::from_code(kraken_hip_copy_buffer_region(
      ctx_, source.raw(), destination.raw(), source_offset, destination_offset, byte_size));
  }
  [[nodiscard]] Status zero_buffer(HipBuffer& buffer, std::size_t byte_size) const {
    return Status::from_code(kraken_hip_zero_buffer(ctx_, buffer.raw(), byte_size));
  }
  // Many ranges from `source` to `destination` in one launch (no counterpart in
  // the reference; at most KRAKEN_COPY_REGIONS_MAX per call).
  [[nodiscard]] Status copy_regions(const HipBuffer& source, HipBuffer& destination,
                                    const kraken_copy_region* regions, std::size_t count) const {
    return Status::from_code(
      kraken_hip_copy_regions(ctx_, source.raw(), destination.raw(), regions, count));
  }

  // Attention (mps_backend.hpp:404-420).
  [[nodiscard]] Status attention_f32_batched_f16_kv(
    const HipBuffer& query, const HipBuffer& key_cache, const HipBuffer& value_cache,
    std::size_t layer, std::size_t start_position, std::size_t tokens,
    std::size_t capacity_tokens, std::size_t heads, std::size_t kv_heads,
    std::size_t head_dim, HipBuffer& output) const {
    return Status::from_code(kraken_hip_attention_f32_batched_f16_kv(
      ctx_, query.raw(), key_cache.raw(), value_cache.raw(), layer, start_position, tokens,
      capacity_tokens, heads, kv_heads, head_dim, output.raw()));
  }
  // attention_f32_batched_f16_kv with an f16 query (no reference counterpart).
  [[nodiscard]] Status attention_f16q_batched_f16_kv(
    const HipBuffer& query, const HipBuffer& key_cache, const HipBuffer& value_cache,
    std::size_t layer, std::size_t start_position, std::size_t tokens,
    std::size_t capacity_tokens, std::size_t heads, std::size_t kv_heads,
    std::size_t head_dim, HipBuffer& output) const {
    return Status::from_code(kraken_hip_attention_f16q_batched_f16_kv(
      ctx_, query.raw(), key_cache.raw(), value_cache.raw(), layer, start_position, tokens,
      capacity_tokens, heads, kv_heads, head_dim, output.raw()));
  }
  [[nodiscard]] Status attention_f32_batched(
    const HipBuffer& query, const HipBuffer& key_cache, const HipBuffer& value_cache,
    std::size_t layer, std::size_t start_position, std::size_t tokens,
    std::size_t capacity_tokens, std::size_t heads, std::size_t kv_heads,
    std::size_t head_dim, HipBuffer& output) const {
    return Status::from_code(kraken_hip_attention_f32_batched(
      ctx_, query.raw(), key_cache.raw(), value_cache.raw(), layer, start_position, tokens,
      capacity_tokens, heads, kv_heads, head_dim, output.raw()));
  }
  // No counterpart in the reference: attention with the full-attention output
  // gate out *= sigmoid(gate) fused (replaces sigmoid + mul after it).
  [[nodiscard]] Status attention_f32_batched_f16_kv_gated(
    const HipBuffer& query, const HipBuffer& key_cache, const HipBuffer& value_cache,
    const HipBuffer& gate, std::size_t layer, std::size_t start_position, std::size_t tokens,
    std::size_t capacity_tokens, std::size_t heads, std::size_t kv_heads,
    std::size_t head_dim, HipBuffer& output) const {
    return Status::from_code(kraken_hip_attention_f32_batched_f16_kv_gated(
      ctx_, query.raw(), key_cache.raw(), value_cache.raw(), gate.raw(), layer, start_position,
      tokens, capacity_tokens, heads, kv_heads, head_dim, output.raw()));
  }

  // Gated delta net (mps_backend.hpp:270-300).
  // Fused full-attention prologue (no MpsContext counterpart; see kraken_hip.h).
  // positions may be an invalid (default) buffer: text positions from
  // mrope_start_position.
  [[nodiscard]] Status qwen35_attention_prologue_f16_kv(
    const HipBuffer& q_gate, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& q_norm, const HipBuffer& k_norm, const HipBuffer& positions,
    std::size_t mrope_start_position, HipBuffer& key_cache, HipBuffer& value_cache,
    std::size_t layer, std::size_t start_position, std::size_t tokens,
    std::size_t capacity_tokens, std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
    std::size_t n_dims, std::size_t section_0, std::size_t section_1, std::size_t section_2,
    std::size_t section_3, float theta, float eps, HipBuffer& query_out,
    HipBuffer& gate_out) const {
    return Status::from_code(kraken_hip_qwen35_attention_prologue_f16_kv(
      ctx_, q_gate.raw(), key.raw(), value.raw(), q_norm.raw(), k_norm.raw(), positions.raw(),
      mrope_start_position, key_cache.raw(), value_cache.raw(), layer, start_position, tokens,
      capacity_tokens, heads, kv_heads, head_dim, n_dims, section_0, section_1, section_2,
      section_3, theta, eps, query_out.raw(), gate_out.raw()));
  }

  // The prologue and the gated attention over the cache (see kraken_hip.h):
  // one launch for a short decode token, else the two calls.
  [[nodiscard]] Status qwen35_attention_prologue_gated_f16_kv(
    const HipBuffer& q_gate, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& q_norm, const HipBuffer& k_norm, const HipBuffer& positions,
    std::size_t mrope_start_position, HipBuffer& key_cache, HipBuffer& value_cache,
    std::size_t layer, std::size_t start_position, std::size_t tokens,
    std::size_t capacity_tokens, std::size_t heads, std::size_t kv_heads, std::size_t head_dim,
    std::size_t n_dims, std::size_t section_0, std::size_t section_1, std::size_t section_2,
    std::size_t section_3, float theta, float eps, HipBuffer& query_out, HipBuffer& gate_out,
    HipBuffer& output) const {
    return Status::from_code(kraken_hip_qwen35_attention_prologue_gated_f16_kv(
      ctx_, q_gate.raw(), key.raw(), value.raw(), q_norm.raw(), k_norm.raw(), positions.raw(),
      mrope_start_position, key_cache.raw(), value_cache.raw(), layer, start_position, tokens,
      capacity_tokens, heads, kv_heads, head_dim, n_dims, section_0, section_1, section_2,
      section_3, theta, eps, query_out.raw(), gate_out.raw(), output.raw()));
  }

  [[nodiscard]] Status gated_delta_net_f32_batched_in_place_at(
    const HipBuffer& query, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& gate, const HipBuffer& beta, HipBuffer& state, std::size_t state_offset,
    std::size_t tokens, std::size_t key_heads, std::size_t value_heads, std::size_t head_dim,
    HipBuffer& output) const {
    return Status::from_code(kraken_hip_gated_delta_net_f32_batched_in_place_at(
      ctx_, query.raw(), key.raw(), value.raw(), gate.raw(), beta.raw(), state.raw(),
      state_offset, tokens, key_heads, value_heads, head_dim, output.raw()));
  }
  [[nodiscard]] Status gated_delta_net_f32_batched_in_place(
    const HipBuffer& query, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& gate, const HipBuffer& beta, HipBuffer& state, std::size_t tokens,
    std::size_t key_heads, std::size_t value_heads, std::size_t head_dim,
    HipBuffer& output) const {
    return Status::from_code(kraken_hip_gated_delta_net_f32_batched_in_place(
      ctx_, query.raw(), key.raw(), value.raw(), gate.raw(), beta.raw(), state.raw(), tokens,
      key_heads, value_heads, head_dim, output.raw()));
  }
  [[nodiscard]] Status gated_delta_net_f32_in_place_at(
    const HipBuffer& query, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& gate, const HipBuffer& beta, HipBuffer& state, std::size_t state_offset,
    std::size_t key_heads, std::size_t value_heads, std::size_t head_dim,
    HipBuffer& output) const {
    return Status::from_code(kraken_hip_gated_delta_net_f32_in_place_at(
      ctx_, query.raw(), key.raw(), value.raw(), gate.raw(), beta.raw(), state.raw(),
      state_offset, key_heads, value_heads, head_dim, output.raw()));
  }

  // Short convolution (mps_backend.hpp:301-330).
  [[nodiscard]] Status ssm_conv_f32(const HipBuffer& input, const HipBuffer& kernel,
                                    std::size_t conv_kernel, std::size_t channels,
                                    std::size_t tokens, std::size_t sequences,
                                    HipBuffer& output) const {
    return Status::from_code(kraken_hip_ssm_conv_f32(ctx_, input.raw(), kernel.raw(),
                                                     conv_kernel, channels, tokens, sequences,
                                                     output.raw()));
  }
  [[nodiscard]] Status build_ssm_conv_state_f32(HipBuffer& state, std::size_t state_offset,
                                                const HipBuffer& input,
                                                std::size_t conv_kernel, std::size_t channels,
                                                std::size_t tokens,
                                                HipBuffer& conv_input) const {
    return Status::from_code(kraken_hip_build_ssm_conv_state_f32(
      ctx_, state.raw(), state_offset, input.raw(), conv_kernel, channels, tokens,
      conv_input.raw()));
  }
  [[nodiscard]] Status ssm_conv1_f32_stateful_at(HipBuffer& state, std::size_t state_offset,
                                                 const HipBuffer& input,
                                                 const HipBuffer& kernel,
                                                 std::size_t conv_kernel,
                                                 std::size_t channels,
                                                 HipBuffer& output) const {
    return Status::from_code(kraken_hip_ssm_conv1_f32_stateful_at(
      ctx_, state.raw(), state_offset, input.raw(), kernel.raw(), conv_kernel, channels,
      output.raw()));
  }

  // No counterparts in the reference: the fused linear-attention prologue
  // (conv state update + conv + SiLU + q/k/v split + q/k L2 norm) and core
  // (gate/beta prepare + recurrence + norm-gated epilogue).
  [[nodiscard]] Status qwen35_conv_split_l2_f32(
    const HipBuffer& qkv, HipBuffer& conv_state, std::size_t state_offset,
    const HipBuffer& conv_kernel_weights, std::size_t conv_kernel, std::size_t tokens,
    std::size_t key_heads, std::size_t value_heads, std::size_t head_dim, float eps,
    HipBuffer& query, HipBuffer& key, HipBuffer& value) const {
    return Status::from_code(kraken_hip_qwen35_conv_split_l2_f32(
      ctx_, qkv.raw(), conv_state.raw(), state_offset, conv_kernel_weights.raw(), conv_kernel,
      tokens, key_heads, value_heads, head_dim, eps, query.raw(), key.raw(), value.raw()));
  }
  [[nodiscard]] Status qwen35_gdn_gated_f32(
    const HipBuffer& query, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& alpha, const HipBuffer& beta_raw, const HipBuffer& dt_bias,
    const HipBuffer& ssm_a, const HipBuffer& z, const HipBuffer& norm_weight,
    HipBuffer& state, std::size_t state_offset, std::size_t tokens, std::size_t key_heads,
    std::size_t value_heads, std::size_t head_dim, float eps, HipBuffer& output) const {
    return Status::from_code(kraken_hip_qwen35_gdn_gated_f32(
      ctx_, query.raw(), key.raw(), value.raw(), alpha.raw(), beta_raw.raw(), dt_bias.raw(),
      ssm_a.raw(), z.raw(), norm_weight.raw(), state.raw(), state_offset, tokens, key_heads,
      value_heads, head_dim, eps, output.raw()));
  }

  // Ragged multi-sequence decode (no counterparts in the reference, which
  // serves one sequence per context): row b of each [sequences][...] operand
  // belongs to sequence b; per-sequence tables are device buffers of uint64
  // element offsets into caller pools and uint32 positions.  A HipBuffer with
  // no data stands for an absent gate.
  [[nodiscard]] Status attention_f32_ragged_f16_kv(
    const HipBuffer& query, const HipBuffer& key_pool, const HipBuffer& value_pool,
    const HipBuffer& gate, const HipBuffer& seq_kv_offsets, const HipBuffer& seq_positions,
    std::size_t sequences, std::size_t max_position, std::size_t heads, std::size_t kv_heads,
    std::size_t head_dim, HipBuffer& output) const {
    return Status::from_code(kraken_hip_attention_f32_ragged_f16_kv(
      ctx_, query.raw(), key_pool.raw(), value_pool.raw(), gate.raw(), seq_kv_offsets.raw(),
      seq_positions.raw(), sequences, max_position, heads, kv_heads, head_dim, output.raw()));
  }
  [[nodiscard]] Status append_kv_ragged_f16(const HipBuffer& key_rows,
                                            const HipBuffer& value_rows, HipBuffer& key_pool,
                                            HipBuffer& value_pool,
                                            const HipBuffer& seq_kv_offsets,
                                            const HipBuffer& seq_positions,
                                            std::size_t sequences,
                                            std::size_t row_size) const {
    return Status::from_code(kraken_hip_append_kv_ragged_f16(
      ctx_, key_rows.raw(), value_rows.raw(), key_pool.raw(), value_pool.raw(),
      seq_kv_offsets.raw(), seq_positions.raw(), sequences, row_size));
  }
  [[nodiscard]] Status gated_delta_net_f32_ragged_decode(
    const HipBuffer& query, const HipBuffer& key, const HipBuffer& value,
    const HipBuffer& gate, const HipBuffer& beta, HipBuffer& state_pool,
    const HipBuffer& seq_state_offsets, std::size_t sequences, std::size_t key_heads,
    std::size_t value_heads, std::size_t head_dim, HipBuffer& output) const {
    return Status::from_code(kraken_hip_gated_delta_net_f32_ragged_decode(
      ctx_, query.raw(), key.raw(), value.raw(), gate.raw(), beta.raw(), state_pool.raw(),
      seq_state_offsets.raw(), sequences, key_heads, value_heads, head_dim, output.raw()));
  }
  [[nodiscard]] Status qwen35_conv_split_l2_ragged_decode_f32(
    const HipBuffer& qkv, HipBuffer& conv_pool, const HipBuffer& seq_conv_offsets,
    const HipBuffer& conv_kernel_weights, std::size_t conv_kernel, std::size_t sequences,
    std::size_t key_heads, std::size_t value_heads, std::size_t head_dim, float eps,
    HipBuffer& query, HipBuffer& key, HipBuffer& value) const {
    return Status::from_code(kraken_hip_qwen35_conv_split_l2_ragged_decode_f32(
      ctx_, qkv.raw(), conv_pool.raw(), seq_conv_offsets.raw(), conv_kernel_weights.raw(),
      conv_kernel, sequences, key_heads, value_heads, head_dim, eps, query.raw(), key.raw(),
      value.raw()));
  }

  // Norms and elementwise ops (mps_backend.hpp:252-376).
  // One decode step of the linear-attention core for many sequences (no
  // MpsContext counterpart; see kraken_hip.h).  dt_bias/ssm_a may be invalid
  // (default) buffers: gate and beta are then already prepared.
  [[nodiscard]] Status qwen35_gdn_layer_ragged_decode_f32(
    const HipBuffer& qkv, HipBuffer& conv_pool, const HipBuffer& seq_conv_offsets,
    const HipBuffer& conv_kernel_weights, std::size_t conv_kernel, const HipBuffer& gate,
    const HipBuffer& beta, const HipBuffer& dt_bias, const HipBuffer& ssm_a, const HipBuffer& z,
    const HipBuffer& norm_weight, HipBuffer& state_pool, const HipBuffer& seq_state_offsets,
    std::size_t sequences, std::size_t key_heads, std::size_t value_heads, std::size_t head_dim,
    float eps, HipBuffer& output) const {
    return Status::from_code(kraken_hip_qwen35_gdn_layer_ragged_decode_f32(
      ctx_, qkv.raw(), conv_pool.raw(), seq_conv_offsets.raw(), conv_kernel_weights.raw(),
      conv_kernel, gate.raw(), beta.raw(), dt_bias.raw(), ssm_a.raw(), z.raw(), norm_weight.raw(),
      state_pool.raw(), seq_state_offsets.raw(), sequences, key_heads, value_heads, head_dim,
      eps, output.raw()));
  }

  // The layer's gated delta rule alone, for a qkv already through the conv
  // (no reference counterpart; see kraken_hip_qwen35_gdn_state_ragged_decode_f32).
  [[nodiscard]] Status qwen35_gdn_state_ragged_decode_f32(
    const HipBuffer& qkv, const HipBuffer& gate, const HipBuffer& beta, const HipBuffer& dt_bias,
    const HipBuffer& ssm_a, const HipBuffer& z, const HipBuffer& norm_weight,
    HipBuffer& state_pool, const HipBuffer& seq_state_offsets, std::size_t sequences,
    std::size_t key_heads, std::size_t value_heads, std::size_t head_dim, float eps,
    HipBuffer& output, HipBuffer& gate_output) const {
    return Status::from_code(kraken_hip_qwen35_gdn_state_ragged_decode_f32(
      ctx_, qkv.raw(), gate.raw(), beta.raw(), dt_bias.raw(), ssm_a.raw(), z.raw(),
      norm_weight.raw(), state_pool.raw(), seq_state_offsets.raw(), sequences, key_heads,
      value_heads, head_dim, eps, output.raw(), gate_output.raw()));
  }

  [[nodiscard]] Status split_qkv_l2_norm_f32_qwen35(
    const HipBuffer& source, HipBuffer& query, HipBuffer& key, HipBuffer& value,
    std::size_t tokens, std::size_t key_heads, std::size_t value_heads, std::size_t head_dim,
    float eps) const {
    return Status::from_code(kraken_hip_split_qkv_l2_norm_f32_qwen35(
      ctx_, source.raw(), query.raw(), key.raw(), value.raw(), tokens, key_heads, value_heads,
      head_dim, eps));
  }
  [[nodiscard]] Status l2_norm_f32_in_place(HipBuffer& values, std::size_t rows,
                                            std::size_t row_size, float eps) const {
    return Status::from_code(
      kraken_hip_l2_norm_f32_in_place(ctx_, values.raw(), rows, row_size, eps));
  }
  [[nodiscard]] Status qk_norm_f32_f32_batched(HipBuffer& values, const HipBuffer& weight,
                                               std::size_t tokens, std::size_t heads,
                                               std::size_t head_dim, float eps) const {
    return Status::from_code(kraken_hip_qk_norm_f32_f32_batched(ctx_, values.raw(), weight.raw(),
                                                                tokens, heads, head_dim, eps));
  }
  [[nodiscard]] Status qwen35_norm_gated_f32_in_place(HipBuffer& values,
                                                      const HipBuffer& weight,
                                                      const HipBuffer& gate,
                                                      std::size_t tokens, std::size_t heads,
                                                      std::size_t head_dim, float eps) const {
    return Status::from_code(kraken_hip_qwen35_norm_gated_f32_in_place(
      ctx_, values.raw(), weight.raw(), gate.raw(), tokens, heads, head_dim, eps));
  }
  [[nodiscard]] Status prepare_qwen35_gdn_gate_beta_f32(HipBuffer& gate, HipBuffer& beta,
                                                        const HipBuffer& gate_bias,
                                                        const HipBuffer& gate_scale,
                                                        std::size_t rows,
                                                        std::size_t row_size) const {
    return Status::from_code(kraken_hip_prepare_qwen35_gdn_gate_beta_f32(
      ctx_, gate.raw(), beta.raw(), gate_bias.raw(), gate_scale.raw(), rows, row_size));
  }
  [[nodiscard]] Status mrope_f32_in_place(HipBuffer& values, const HipBuffer& positions,
                                          std::size_t tokens, std::size_t heads,
                                          std::size_t head_dim, std::size_t n_dims,
                                          std::size_t section_0, std::size_t section_1,
                                          std::size_t section_2, std::size_t section_3,
                                          float theta) const {
    return Status::from_code(kraken_hip_mrope_f32_in_place(
      ctx_, values.raw(), positions.raw(), tokens, heads, head_dim, n_dims, section_0,
      section_1, section_2, section_3, theta));
  }
  [[nodiscard]] Status copy_f32_rows_to_f16(const HipBuffer& source, HipBuffer& destination,
                                            std::size_t rows, std::size_t row_size,
                                            std::size_t source_stride,
                                            std::size_t source_offset,
                                            std::size_t destination_stride,
                                            std::size_t destination_offset) const {
    return Status::from_code(kraken_hip_copy_f32_rows_to_f16(
      ctx_, source.raw(), destination.raw(), rows, row_size, source_stride, source_offset,
      destination_stride, destination_offset));
  }
  [[nodiscard]] Status copy_f32_rows(const HipBuffer& source, HipBuffer& destination,
                                     std::size_t rows, std::size_t row_size,
                                     std::size_t source_stride, std::size_t source_offset,
                                     std::size_t destination_stride,
                                     std::size_t destination_offset) const {
    return Status::from_code(kraken_hip_copy_f32_rows(ctx_, source.raw(), destination.raw(),
                                                      rows, row_size, source_stride,
                                                      source_offset, destination_stride,
                                                      destination_offset));
  }
  [[nodiscard]] Status copy_f16_rows(const HipBuffer& source, HipBuffer& destination,
                                     std::size_t rows, std::size_t row_size,
                                     std::size_t source_stride, std::size_t source_offset,
                                     std::size_t destination_stride,
                                     std::size_t destination_offset) const {
    return Status::from_code(kraken_hip_copy_f16_rows(ctx_, source.raw(), destination.raw(),
                                                      rows, row_size, source_stride,
                                                      source_offset, destination_stride,
                                                      destination_offset));
  }
  [[nodiscard]] Status sigmoid_f32_in_place(HipBuffer& values, std::size_t size) const {
    return Status::from_code(kraken_hip_sigmoid_f32_in_place(ctx_, values.raw(), size));
  }
  [[nodiscard]] Status softplus_f32_in_place(HipBuffer& values, std::size_t size) const {
    return Status::from_code(kraken_hip_softplus_f32_in_place(ctx_, values.raw(), size));
  }
  [[nodiscard]] Status silu_f32_in_place(HipBuffer& values, std::size_t size) const {
    return Status::from_code(kraken_hip_silu_f32_in_place(ctx_, values.raw(), size));
  }
  [[nodiscard]] Status mul_f32_in_place(HipBuffer& target, const HipBuffer& rhs,
                                        std::size_t size) const {
    return Status::from_code(kraken_hip_mul_f32_in_place(ctx_, target.raw(), rhs.raw(), size));
  }
  [[nodiscard]] Status add_f32_row_in_place(HipBuffer& target, const HipBuffer& row,
                                            std::size_t rows, std::size_t row_size) const {
    return Status::from_code(
      kraken_hip_add_f32_row_in_place(ctx_, target.raw(), row.raw(), rows, row_size));
  }
  [[nodiscard]] Status mul_f32_row_in_place(HipBuffer& target, const HipBuffer& row,
                                            std::size_t rows, std::size_t row_size) const {
    return Status::from_code(
      kraken_hip_mul_f32_row_in_place(ctx_, target.raw(), row.raw(), rows, row_size));
  }
  [[nodiscard]] Status add_f32_in_place(HipBuffer& target, const HipBuffer& delta,
                                        std::size_t size) const {
    return Status::from_code(kraken_hip_add_f32_in_place(ctx_, target.raw(), delta.raw(), size));
  }
  [[nodiscard]] Status silu_mul_f32_in_place(HipBuffer& gate, const HipBuffer& up,
                                             std::size_t size) const {
    return Status::from_code(kraken_hip_silu_mul_f32_in_place(ctx_, gate.raw(), up.raw(), size));
  }
  [[nodiscard]] Status rms_norm_f32_f32_batched(const HipBuffer& input, const HipBuffer& weight,
                                                std::size_t tokens, std::size_t size, float eps,
                                                HipBuffer& output) const {
    return Status::from_code(kraken_hip_rms_norm_f32_f32_batched(
      ctx_, input.raw(), weight.raw(), tokens, size, eps, output.raw()));
  }

  // K-quant projections (mps_backend.hpp:134-226).  matvec_*_f32 takes and
  // returns host vectors through temporary device buffers, as the reference's
  // overload does (mps_backend.mm:6456-6492).
  [[nodiscard]] Result<std::vector<float>> matvec_q4_k_f32(const HipBuffer& weight,
                                                        std::size_t rows, std::size_t cols,
                                                        const std::vector<float>& input) const {
    return host_matvec(&kraken_hip_matvec_q4_k_f32_device, "HIP Q4_K", weight, rows, cols, input);
  }
  [[nodiscard]] Status matvec_q4_k_f32_device(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, const HipBuffer& input,
                                          HipBuffer& output) const {
    return Status::from_code(kraken_hip_matvec_q4_k_f32_device(ctx_, weight.raw(), rows, cols,
                                                              input.raw(), output.raw()));
  }
  [[nodiscard]] Status matvec_q4_k_f32_top1(const HipBuffer& weight, std::size_t rows,
                                        std::size_t cols, const HipBuffer& input,
                                        HipBuffer& token_output,
                                        HipBuffer& probability_output) const {
    return Status::from_code(kraken_hip_matvec_q4_k_f32_top1(
      ctx_, weight.raw(), rows, cols, input.raw(), token_output.raw(), probability_output.raw()));
  }
  [[nodiscard]] Status matvec_q4_k_f32_argmax(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, const HipBuffer& input,
                                          HipBuffer& token_output) const {
    return Status::from_code(kraken_hip_matvec_q4_k_f32_argmax(ctx_, weight.raw(), rows, cols,
                                                              input.raw(), token_output.raw()));
  }
  [[nodiscard]] Status matmul_q4_k_f32_device(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, std::size_t tokens,
                                          const HipBuffer& input, HipBuffer& output) const {
    return Status::from_code(kraken_hip_matmul_q4_k_f32_device(ctx_, weight.raw(), rows, cols,
                                                              tokens, input.raw(), output.raw()));
  }
  [[nodiscard]] Status dequantize_row_q4_k_f32(const HipBuffer& weight, std::size_t row,
                                           std::size_t cols, HipBuffer& output) const {
    return Status::from_code(
      kraken_hip_dequantize_row_q4_k_f32(ctx_, weight.raw(), row, cols, output.raw()));
  }
  [[nodiscard]] Status dequantize_rows_q4_k_f32(const HipBuffer& weight, std::size_t rows,
                                            const HipBuffer& row_ids, std::size_t tokens,
                                            std::size_t cols, HipBuffer& output) const {
    return Status::from_code(kraken_hip_dequantize_rows_q4_k_f32(
      ctx_, weight.raw(), rows, row_ids.raw(), tokens, cols, output.raw()));
  }
  [[nodiscard]] Result<std::vector<float>> matvec_q5_k_f32(const HipBuffer& weight,
                                                        std::size_t rows, std::size_t cols,
                                                        const std::vector<float>& input) const {
    return host_matvec(&kraken_hip_matvec_q5_k_f32_device, "HIP Q5_K", weight, rows, cols, input);
  }
  [[nodiscard]] Status matvec_q5_k_f32_device(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, const HipBuffer& input,
                                          HipBuffer& output) const {
    return Status::from_code(kraken_hip_matvec_q5_k_f32_device(ctx_, weight.raw(), rows, cols,
                                                              input.raw(), output.raw()));
  }
  [[nodiscard]] Status matvec_q5_k_f32_top1(const HipBuffer& weight, std::size_t rows,
                                        std::size_t cols, const HipBuffer& input,
                                        HipBuffer& token_output,
                                        HipBuffer& probability_output) const {
    return Status::from_code(kraken_hip_matvec_q5_k_f32_top1(
      ctx_, weight.raw(), rows, cols, input.raw(), token_output.raw(), probability_output.raw()));
  }
  [[nodiscard]] Status matvec_q5_k_f32_argmax(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, const HipBuffer& input,
                                          HipBuffer& token_output) const {
    return Status::from_code(kraken_hip_matvec_q5_k_f32_argmax(ctx_, weight.raw(), rows, cols,
                                                              input.raw(), token_output.raw()));
  }
  [[nodiscard]] Status matmul_q5_k_f32_device(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, std::size_t tokens,
                                          const HipBuffer& input, HipBuffer& output) const {
    return Status::from_code(kraken_hip_matmul_q5_k_f32_device(ctx_, weight.raw(), rows, cols,
                                                              tokens, input.raw(), output.raw()));
  }
  [[nodiscard]] Status dequantize_row_q5_k_f32(const HipBuffer& weight, std::size_t row,
                                           std::size_t cols, HipBuffer& output) const {
    return Status::from_code(
      kraken_hip_dequantize_row_q5_k_f32(ctx_, weight.raw(), row, cols, output.raw()));
  }
  [[nodiscard]] Status dequantize_rows_q5_k_f32(const HipBuffer& weight, std::size_t rows,
                                            const HipBuffer& row_ids, std::size_t tokens,
                                            std::size_t cols, HipBuffer& output) const {
    return Status::from_code(kraken_hip_dequantize_rows_q5_k_f32(
      ctx_, weight.raw(), rows, row_ids.raw(), tokens, cols, output.raw()));
  }
  [[nodiscard]] Result<std::vector<float>> matvec_q6_k_f32(const HipBuffer& weight,
                                                        std::size_t rows, std::size_t cols,
                                                        const std::vector<float>& input) const {
    return host_matvec(&kraken_hip_matvec_q6_k_f32_device, "HIP Q6_K", weight, rows, cols, input);
  }
  [[nodiscard]] Status matvec_q6_k_f32_device(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, const HipBuffer& input,
                                          HipBuffer& output) const {
    return Status::from_code(kraken_hip_matvec_q6_k_f32_device(ctx_, weight.raw(), rows, cols,
                                                              input.raw(), output.raw()));
  }
  [[nodiscard]] Status matvec_q6_k_f32_top1(const HipBuffer& weight, std::size_t rows,
                                        std::size_t cols, const HipBuffer& input,
                                        HipBuffer& token_output,
                                        HipBuffer& probability_output) const {
    return Status::from_code(kraken_hip_matvec_q6_k_f32_top1(
      ctx_, weight.raw(), rows, cols, input.raw(), token_output.raw(), probability_output.raw()));
  }
  [[nodiscard]] Status matvec_q6_k_f32_argmax(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, const HipBuffer& input,
                                          HipBuffer& token_output) const {
    return Status::from_code(kraken_hip_matvec_q6_k_f32_argmax(ctx_, weight.raw(), rows, cols,
                                                              input.raw(), token_output.raw()));
  }
  [[nodiscard]] Status matmul_q6_k_f32_device(const HipBuffer& weight, std::size_t rows,
                                          std::size_t cols, std::size_t tokens,
                                          const HipBuffer& input, HipBuffer& output) const {
    return Status::from_code(kraken_hip_matmul_q6_k_f32_device(ctx_, weight.raw(), rows, cols,
                                                              tokens, input.raw(), output.raw()));
  }
  [[nodiscard]] Status dequantize_row_q6_k_f32(const HipBuffer& weight, std::size_t row,
                                           std::size_t cols, HipBuffer& output) const {
    return Status::from_code(
      kraken_hip_dequantize_row_q6_k_f32(ctx_, weight.raw(), row, cols, output.raw()));
  }
  [[nodiscard]] Status dequantize_rows_q6_k_f32(const HipBuffer& weight, std::size_t rows,
                                            const HipBuffer& row_ids, std::size_t tokens,
                                            std::size_t cols, HipBuffer& output) const {
    return Status::from_code(kraken_hip_dequantize_rows_q6_k_f32(
      ctx_, weight.raw(), rows, row_ids.raw(), tokens, cols, output.raw()));
  }

  // No counterpart in the reference: the one-token K-quant GEMV with RMSNorm or
  // SwiGLU on its input and a residual add on its output (empty buffers when
  // unused), and the top-1 LM head with the output norm folded in.
  [[nodiscard]] Status kquant_matvec_fused_f32(std::uint32_t ggml_type, const HipBuffer& weight,
                                               std::size_t rows, std::size_t cols,
                                               const HipBuffer& input,
                                               const HipBuffer& norm_weight, float eps,
                                               const HipBuffer& up, const HipBuffer& residual,
                                               HipBuffer& output) const {
    return Status::from_code(kraken_hip_kquant_matvec_fused_f32(
      ctx_, ggml_type, weight.raw(), rows, cols, input.raw(), norm_weight.raw(), eps, up.raw(),
      residual.raw(), output.raw()));
  }
  // A K-quant matmul of more than 8 tokens with SwiGLU on its input (up given)
  // and a residual add (which may be `output`) folded in; see kraken_hip.h.
  [[nodiscard]] Status kquant_matmul_fused_f32(std::uint32_t ggml_type, const HipBuffer& weight,
                                               std::size_t rows, std::size_t cols,
                                               std::size_t tokens, const HipBuffer& input,
                                               const HipBuffer& up, const HipBuffer& residual,
                                               HipBuffer& output) const {
    return Status::from_code(kraken_hip_kquant_matmul_fused_f32(ctx_, ggml_type, weight.raw(),
                                                                rows, cols, tokens, input.raw(),
                                                                up.raw(), residual.raw(),
                                                                output.raw()));
  }
  // Up to four K-quant matmuls over one input [tokens][cols] (one launch when
  // their type allows it; see kraken_hip.h).
  [[nodiscard]] Status kquant_matmul_multi_f32(std::size_t count, const std::uint32_t* ggml_types,
                                               const HipBuffer* const* weights,
                                               const std::size_t* rows, std::size_t cols,
                                               std::size_t tokens, const HipBuffer& input,
                                               HipBuffer* const* outputs) const {
    kraken_buffer w[4], out[4];
    for (std::size_t i = 0; i < count && i < 4; ++i) {
      w[i] = weights[i]->raw();
      out[i] = outputs[i]->raw();
    }
    return Status::from_code(kraken_hip_kquant_matmul_multi_f32(ctx_, count, ggml_types, w, rows,
                                                                cols, tokens, input.raw(), out));
  }
  // Up to four fused GEMVs over one input in one launch; entries of `weights`,
  // `outputs` and `residuals` (nullptr for none) per matrix.
  [[nodiscard]] Status kquant_matvec_multi_f32(std::size_t count, const std::uint32_t* ggml_types,
                                               const HipBuffer* const* weights,
                                               const std::size_t* rows, std::size_t cols,
                                               const HipBuffer& input,
                                               const HipBuffer& norm_weight, float eps,
                                               const HipBuffer& up,
                                               const HipBuffer* const* residuals,
                                               HipBuffer* const* outputs) const {
    kraken_buffer w[4], res[4], out[4];
    for (std::size_t i = 0; i < count && i < 4; ++i) {
      w[i] = weights[i]->raw();
      res[i] = residuals[i] != nullptr ? residuals[i]->raw() : kraken_buffer{nullptr, 0};
      out[i] = outputs[i]->raw();
    }
    return Status::from_code(kraken_hip_kquant_matvec_multi_f32(
      ctx_, count, ggml_types, w, rows, cols, input.raw(), norm_weight.raw(), eps, up.raw(), res,
      out));
  }
  // kquant_matvec_multi_f32 whose matrix 0 rows take the conv prologue (no
  // reference counterpart; see kraken_hip_kquant_matvec_multi_conv_f32).
  [[nodiscard]] Status kquant_matvec_multi_conv_f32(
    std::size_t count, const std::uint32_t* ggml_types, const HipBuffer* const* weights,
    const std::size_t* rows, std::size_t cols, const HipBuffer& input,
    const HipBuffer& norm_weight, float eps, HipBuffer* const* outputs, HipBuffer& conv_pool,
    const HipBuffer& conv_offset, const HipBuffer& conv_kernel_weights,
    std::size_t conv_kernel) const {
    kraken_buffer w[4], out[4];
    for (std::size_t i = 0; i < count && i < 4; ++i) {
      w[i] = weights[i]->raw();
      out[i] = outputs[i]->raw();
    }
    return Status::from_code(kraken_hip_kquant_matvec_multi_conv_f32(
      ctx_, count, ggml_types, w, rows, cols, input.raw(), norm_weight.raw(), eps, out,
      conv_pool.raw(), conv_offset.raw(), conv_kernel_weights.raw(), conv_kernel));
  }
  // The output projection GEMV with the norm-gated epilogue finished on its
  // input (no reference counterpart; see kraken_hip_kquant_matvec_head_norm_f32).
  [[nodiscard]] Status kquant_matvec_head_norm_f32(
    std::uint32_t ggml_type, const HipBuffer& weight, std::size_t rows, std::size_t cols,
    const HipBuffer& input, const HipBuffer& gate_factor, std::size_t head_dim, float eps,
    const HipBuffer& residual, HipBuffer& output) const {
    return Status::from_code(kraken_hip_kquant_matvec_head_norm_f32(
      ctx_, ggml_type, weight.raw(), rows, cols, input.raw(), gate_factor.raw(), head_dim, eps,
      residual.raw(), output.raw()));
  }
  [[nodiscard]] Status kquant_top1_fused_f32(std::uint32_t ggml_type, const HipBuffer& weight,
                                             std::size_t rows, std::size_t cols,
                                             const HipBuffer& input, const HipBuffer& norm_weight,
                                             float eps, HipBuffer& token_output,
                                             HipBuffer& probability_output) const {
    return Status::from_code(kraken_hip_kquant_top1_fused_f32(
      ctx_, ggml_type, weight.raw(), rows, cols, input.raw(), norm_weight.raw(), eps,
      token_output.raw(), probability_output.raw()));
  }

  // Device argmax (mps_backend.hpp:384-390).
  [[nodiscard]] Status argmax_f32_i32(const HipBuffer& values, std::size_t size,
                                      HipBuffer& output) const {
    return Status::from_code(kraken_hip_argmax_f32_i32(ctx_, values.raw(), size, output.raw()));
  }
  [[nodiscard]] Status argmax_prob_f32_i32(const HipBuffer& values, std::size_t size,
                                           HipBuffer& token_output,
                                           HipBuffer& probability_output) const {
    return Status::from_code(kraken_hip_argmax_prob_f32_i32(
      ctx_, values.raw(), size, token_output.raw(), probability_output.raw()));
  }

 private:
  explicit HipContext(kraken_hip_context* raw) : ctx_(raw) {}

  using MatvecEntry = int (*)(kraken_hip_context*, kraken_buffer, std::size_t, std::size_t,
                              kraken_buffer, kraken_buffer);

  // The host-vector matvec: input size check, buffers, copy in, run, copy out.
  [[nodiscard]] Result<std::vector<float>> host_matvec(MatvecEntry entry, const char* name,
                                                       const HipBuffer& weight,
                                                       std::size_t rows, std::size_t cols,
                                                       const std::vector<float>& input) const {
    if (input.size() != cols) {
      return Status::invalid_argument(std::string(name) +
                                      " matvec input size does not match cols");
    }
    if (rows == 0 || cols == 0 || rows > SIZE_MAX / sizeof(float)) {
      return Status::invalid_argument(std::string(name) +
                                      " matvec rows and cols must be greater than zero");
    }
    auto in = make_buffer(cols * sizeof(float));
    if (!in.is_ok()) {
      return in.status();
    }
    auto out = make_buffer(rows * sizeof(float));
    if (!out.is_ok()) {
      return out.status();
    }
    Status s = copy_to_buffer(in.value(), input.data(), cols * sizeof(float));
    if (!s.is_ok()) {
      return s;
    }
    s = Status::from_code(entry(ctx_, weight.raw(), rows, cols, in.value().raw(),
                                out.value().raw()));
    if (!s.is_ok()) {
      return s;
    }
    std::vector<float> output(rows);
    s = copy_from_buffer(out.value(), output.data(), rows * sizeof(float));
    if (!s.is_ok()) {
      return s;
    }
    return output;
  }

  kraken_hip_context* ctx_{nullptr};
};

}  // namespace kraken::hip
