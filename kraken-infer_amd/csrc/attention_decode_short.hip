// Short-split MFMA decode kernel (head_dim 256, f16 cache), in its own
// translation unit: it keeps its MFMA accumulators in architectural VGPRs
// (built with -mllvm -amdgpu-mfma-vgpr-form), so the softmax rescale and the
// epilogue read them without AGPR copies.
//
// Semantics: reference MSL attention_f32_batched_f16_kv (mps_backend.mm:
// 2943-3008) with the output gate of qwen35_runtime.cpp:3347-3355, as in
// attention_decode.hip, whose merge pass combines the split partials.
#include <hip/hip_runtime.h>

#include "attention_decode_internal.hpp"
#include "device_common.hpp"

namespace kraken {
namespace decode {
namespace {

// ---------------------------------------------------------------------------
// Short-split MFMA kernel: head_dim 256, f16 cache, G <= 4, one sequence, for
// splits of a few dozen keys (batch-1 decode, where a split is what one CU
// reads).  There the step is bounded by latency, not by bandwidth, so every
// load of the split is issued before anything else: a wave's K tile goes
// straight into the MFMA A-fragment registers (lane (key r16, kq) loads dims
// 32 s + 8 kq .. + 7 of step s) and its V tile into registers that are then
// written to the wave's LDS region for the transposing V^T reads; the query
// is loaded after them.  The math is the MFMA kernel's (split fp16 query and
// probabilities, lazy rescale, same partial format); a wave with more than one
// tile loads its next tile while it computes the current one.  The query
// fragments stay in LDS and are read per tile, which leaves the registers for
// the second (lo) output accumulator.
// ---------------------------------------------------------------------------
//
// kFold (one decode token, one split): the attention prologue runs inside the
// workgroup.  Its raw inputs are loaded first, then the K/V tile; waves 0..G-1
// normalise and rotate the workgroup's query heads into LDS (read by the
// query conversion in place of p.query), one wave does the K head and one the
// V head: f16 into the cache row at start_position and into LDS, from where
// the wave holding that row's tile puts it in place of the loaded row (the
// cache row is written by this same workgroup, so what the load returned for
// it is not used).  The output gate comes from the second half of each q_gate
// head, loaded at the start.
// ---------------------------------------------------------------------------
constexpr int kSWaves = 4;

template <int G, bool kFold>
__global__ __launch_bounds__(64 * kSWaves) void attention_decode_short_kernel(DecodeParams p,
                                                                              PrologueFold f) {
  static_assert(G == 1 || G == 2 || G == 4, "query heads per KV head (rows 0..3 of a tile)");
  __shared__ __attribute__((aligned(16))) half_t s_v[kSWaves][kMTileHalfs];
  // Query fragments (hi, lo) per MFMA step, converted cooperatively.
  __shared__ __attribute__((aligned(16))) half8_t s_q[8][2][64];
  __shared__ float s_m[kSWaves][G];
  __shared__ float s_l[kSWaves][G];
  // kFold: the new K and V rows (f16), read inside the tile loop.
  __shared__ __attribute__((aligned(16))) half_t s_new[kFold ? 2 : 1][kFold ? kMD : 8];
  static_assert(sizeof(float) * kSWaves * G * kMD <= sizeof(s_v), "merge area");
  float(*s_o)[G * kMD] = reinterpret_cast<float(*)[G * kMD]>(&s_v[0][0]);
  // kFold: the prepared query heads, in the V area before the tile loop uses it.
  float(*s_qf)[kMD] = reinterpret_cast<float(*)[kMD]>(&s_v[0][0]);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const uint32_t split = blockIdx.x;
  const uint32_t kvh = blockIdx.y;
  const uint32_t token = blockIdx.z;
  const uint32_t n_keys = token_keys(nullptr, p.start_position, token);
  const uint32_t key_begin = split * p.keys_per_split;
  if (key_begin >= n_keys) {
    return;  // empty split (whole workgroup)
  }
  const uint32_t count = min(n_keys, key_begin + p.keys_per_split) - key_begin;
  const size_t row_stride = (size_t)p.kv_heads * kMD;
  const uint32_t row_bytes = (uint32_t)(row_stride * sizeof(half_t));
  const size_t first = ((size_t)p.layer * p.capacity_tokens + key_begin) * row_stride +
                       (size_t)kvh * kMD;
  // Rows at or past the split's end read as zeros (resource range check).
  const __amdgpu_buffer_rsrc_t krs =
    make_buffer_rsrc(static_cast<const half_t*>(p.key_cache) + first, count * row_bytes);
  const __amdgpu_buffer_rsrc_t vrs =
    make_buffer_rsrc(static_cast<const half_t*>(p.value_cache) + first, count * row_bytes);
  const uint32_t ntiles = (count + kMTile - 1) / kMTile;

  // The query first: loads retire in issue order, so its conversion below
  // waits only for the query while the K/V tile is still in flight.  Wave w
  // converts steps 2 w and 2 w + 1: lane (head r16, kq) holds dims
  // 32 s + 8 kq .. + 7 of step s, scaled into the log2 domain.
  float4 qraw[2][2];
  const int qg = r16 < G ? r16 : 0;
  const float qscale = r16 < G ? p.scale_log2 : 0.0f;
  // kFold: the prologue's inputs in the same position (wave k_wave takes the
  // K head, v_wave the V head, waves below G a query head each).
  constexpr int k_wave = G < 4 ? G : 0;
  constexpr int v_wave = G < 3 ? G + 1 : 1;
  float hv[4], hw[4], kv[4], kw[4], gate_v[G];
  int32_t rpos[4];
  if constexpr (kFold) {
    if (wave < G) {
      load_head(f.q_gate + (size_t)(kvh * G + wave) * 2u * kMD, f.q_norm, kMD, lane, hv, hw);
    }
    if (wave == k_wave) {
      load_head(f.key + (size_t)kvh * kMD, f.k_norm, kMD, lane, kv, kw);
    }
    if (wave == v_wave) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kv[i] = f.value[(size_t)kvh * kMD + lane + 64 * i];
      }
    }
    // Output element tid of head k (the merge's index) and its gate.
#pragma unroll
    for (int k = 0; k < G; ++k) {
      gate_v[k] = f.q_gate[(size_t)(kvh * G + k) * 2u * kMD + kMD + tid];
    }
    rope_positions(f.rope, 0, rpos);
  } else {
    const float* qh = p.query + ((size_t)token * p.heads + kvh * G + qg) * kMD + 8 * kq;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int s = 2 * wave + i;
      qraw[i][0] = *reinterpret_cast<const float4*>(qh + 32 * s);
      qraw[i][1] = *reinterpret_cast<const float4*>(qh + 32 * s + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  half8_t kf[8];
  u32x4_t vr[8];
  const uint32_t k_off = (uint32_t)r16 * row_bytes + 16u * (uint32_t)kq;
  const uint32_t v_off = (uint32_t)(lane >> 5) * row_bytes + 16u * (uint32_t)(lane & 31);
  auto load_k = [&](uint32_t t) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      kf[s] = __builtin_bit_cast(half8_t,
                                 buffer_load_nt_b128(krs, t * kMTile * row_bytes + k_off + 64u * s));
    }
  };
  auto load_v = [&](uint32_t t) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      vr[c] = buffer_load_nt_b128(vrs, (t * kMTile + 2u * c) * row_bytes + v_off);
    }
  };
  uint32_t t = (uint32_t)wave;
  if (t < ntiles) {
    load_k(t);
    load_v(t);
  }
  __builtin_amdgcn_sched_barrier(0);

  const uint32_t new_key = p.start_position;  // kFold: the appended row
  if constexpr (kFold) {
    const size_t cache_row =
      ((size_t)p.layer * p.capacity_tokens + new_key) * row_stride + (size_t)kvh * kMD;
    if (wave < G || wave == k_wave) {
      double sn[4], cs[4];
      rope_angles(f.rope, rpos, lane, sn, cs);
      float r[4];
      if (wave < G) {
        norm_rope(hv, hw, kMD, f.eps, f.rope.n_dims, sn, cs, lane, r);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s_qf[wave][lane + 64 * i] = r[i];
        }
      }
      if (wave == k_wave) {
        norm_rope(kv, kw, kMD, f.eps, f.rope.n_dims, sn, cs, lane, r);
        half_t* dst = static_cast<half_t*>(const_cast<void*>(p.key_cache)) + cache_row;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const half_t h = static_cast<half_t>(r[i]);
          s_new[0][lane + 64 * i] = h;
          dst[lane + 64 * i] = h;
        }
      }
    }
    if (wave == v_wave) {
      half_t* dst = static_cast<half_t*>(const_cast<void*>(p.value_cache)) + cache_row;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const half_t h = static_cast<half_t>(kv[i]);
        s_new[1][lane + 64 * i] = h;
        dst[lane + 64 * i] = h;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float* qh = &s_qf[qg][32 * (2 * wave + i) + 8 * kq];
      qraw[i][0] = *reinterpret_cast<const float4*>(qh);
      qraw[i][1] = *reinterpret_cast<const float4*>(qh + 4);
    }
  }

  // Query fragments (B operand of S^T) in the split fp16 form (split_f16:
  // hi, and lo scaled by 2^11), so that K (exact in f16) times hi plus 2^-11
  // times K lo reproduces the f32 product to about 2^-21 relative.
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float v[8] = {qraw[i][0].x, qraw[i][0].y, qraw[i][0].z, qraw[i][0].w,
                        qraw[i][1].x, qraw[i][1].y, qraw[i][1].z, qraw[i][1].w};
    half8_t hi8, lo8;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      half_t hi, lo;
      split_f16(v[j] * qscale, hi, lo);
      hi8[j] = hi;
      lo8[j] = lo;
    }
    s_q[2 * wave + i][0][lane] = hi8;
    s_q[2 * wave + i][1][lane] = lo8;
  }
  __syncthreads();  // (kFold: also every wave is done reading s_qf)

  float m[G];  // wave-uniform reference max per head (log2 domain)
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
  }
  // This lane's share of head r16's denominator, summed with Kahan's
  // compensation (lcomp): a long split adds thousands of small weights to a sum
  // near 1, where plain fp32 addition would drop a systematic part of each.
  float lpart = 0.0f;
  float lcomp = 0.0f;
  // O tile n: lane l holds dim 16 n + l % 16 of heads 4 (l / 16) + r; o from
  // the hi probabilities, olo from the lo ones (scaled by 2^11).
  float4v_t o[16], olo[16];
#pragma unroll
  for (int n = 0; n < 16; ++n) {
    o[n] = float4v_t{0.f, 0.f, 0.f, 0.f};
    olo[n] = float4v_t{0.f, 0.f, 0.f, 0.f};
  }
  half_t* vs = &s_v[wave][0];
  for (; t < ntiles; t += kSWaves) {
    if constexpr (kFold) {
      if (t == new_key / kMTile) {  // wave-uniform: put the new row in place
        const uint32_t row = new_key % kMTile;
        const half8_t* nk = reinterpret_cast<const half8_t*>(&s_new[0][0]);
        const u32x4_t* nv = reinterpret_cast<const u32x4_t*>(&s_new[1][0]);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          kf[s] = (uint32_t)r16 == row ? nk[4 * s + kq] : kf[s];
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          vr[c] = 2u * c + (uint32_t)(lane >> 5) == row ? nv[lane & 31] : vr[c];
        }
      }
    }
    // V rows of tile t into the wave's LDS region, 16-byte chunks XOR-swizzled
    // by 2 (row & 3) so that the transposing reads are free of bank conflicts.
    // The region's previous reads were consumed by last tile's MFMAs.
    asm volatile("" ::: "memory");
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint32_t row = 2u * c + (uint32_t)(lane >> 5);
      const uint32_t chunk = (uint32_t)(lane & 31);
      *reinterpret_cast<u32x4_t*>(vs + row * kMD + 8 * (chunk ^ (2u * (row & 3u)))) = vr[c];
    }
    asm volatile("" ::: "memory");
    const bool more = t + kSWaves < ntiles;
    if (more) {
      load_v(t + kSWaves);
    }

    // S^T = K Q^T (keys x heads): the hi and the lo chain, then combined.
    float4v_t shi = {0.f, 0.f, 0.f, 0.f};
    float4v_t slo = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      shi = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[s], s_q[s][0][lane], shi, 0, 0, 0);
      slo = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[s], s_q[s][1][lane], slo, 0, 0, 0);
    }
    if (more) {
      load_k(t + kSWaves);
    }
    float4v_t sacc;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sacc[r] = fmaf(slo[r], kLoUnscale, shi[r]);
    }

    // Softmax: lane holds keys 16 t + 4 kq + r of head r16.
    float sc[4];
    bool valid[4];
    float cmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      valid[r] = r16 < G && kMTile * t + 4u * kq + r < count;
      sc[r] = valid[r] ? sacc[r] : -INFINITY;
      cmax = fmaxf(cmax, sc[r]);
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    float corr_lane = 1.0f;
    float m_lane = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float bm = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                   __builtin_bit_cast(int, cmax), g));
      if (bm > m[g] + kRescaleSlack) {  // wave-uniform
        // Before the head's first valid tile o and l are zero: no rescale.
        if (m[g] != -INFINITY) {
          const float corr = fast_exp2(m[g] - bm);
#pragma unroll
          for (int n = 0; n < 16; ++n) {
            o[n][g] *= corr;  // head g is row g: register g of lanes 0..15
            olo[n][g] *= corr;
          }
          corr_lane = r16 == g ? corr : corr_lane;
        }
        m[g] = bm;
      }
      m_lane = r16 == g ? m[g] : m_lane;
    }
    lpart *= corr_lane;
    lcomp *= corr_lane;
    half4_t phi, plo;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float pr = valid[r] ? fast_exp2(sc[r] - m_lane) : 0.0f;
      kahan_add(lpart, lcomp, pr);
      half_t h, l;
      split_f16(pr, h, l);
      phi[r] = h;
      plo[r] = l;
    }

    // O += P V: lane 4 e + q of group kq points at row 4 kq + e, columns
    // 16 n + 4 q .. + 3; the transposing read returns column 16 n + l % 16
    // of rows 4 kq .. 4 kq + 3.
    const int vrow = 4 * kq + (r16 >> 2);
    const int q = r16 & 3;
    const half_t* vrow_p = vs + vrow * kMD + 4 * (q & 1);
    const int vswz = 2 * (vrow & 3);
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      const half4_t vf = read_tr16(vrow_p + 8 * ((2 * n + (q >> 1)) ^ vswz));
      o[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(phi, vf, o[n], 0, 0, 0);
      olo[n] = __builtin_amdgcn_mfma_f32_16x16x16f16(plo, vf, olo[n], 0, 0, 0);
    }
  }

  // Wave partial: head r16's denominator over the four lane groups.
  float lw = lpart - lcomp;
  lw += __shfl_xor(lw, 16, 64);
  lw += __shfl_xor(lw, 32, 64);
  __syncthreads();  // every wave is done with its V region
  if (lane < G) {
    s_l[wave][lane] = lw;
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      s_m[wave][g] = m[g];
    }
  }
  if (lane < 16) {
#pragma unroll
    for (int n = 0; n < 16; ++n) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        s_o[wave][g * kMD + 16 * n + lane] = fmaf(olo[n][g], kLoUnscale, o[n][g]);
      }
    }
  }
  __syncthreads();

  // Workgroup merge of the wave partials (waves without a tile hold m = -inf).
  constexpr int kThreads = 64 * kSWaves;
  constexpr int kOutPerThread = G * kMD / kThreads;
  const size_t tk = (size_t)token * p.kv_heads + kvh;
  float* po = p.part_o + (tk * p.splits + split) * (size_t)(G * kMD);
  float* pml = p.part_ml + (tk * p.splits + split) * (size_t)(G * 2);
#pragma unroll
  for (int k = 0; k < kOutPerThread; ++k) {
    const int idx = tid + k * kThreads;
    const int g = idx / kMD;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSWaves; ++w) {
      mx = fmaxf(mx, s_m[w][g]);
    }
    float acc = 0.0f;
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < kSWaves; ++w) {
      const float wt = s_m[w][g] == -INFINITY ? 0.0f : fast_exp2(s_m[w][g] - mx);
      acc = fmaf(wt, s_o[w][idx], acc);
      den = fmaf(wt, s_l[w][g], den);
    }
    if constexpr (kFold) {
      const size_t out_index = ((size_t)kvh * G + k) * kMD + tid;
      float r = den == 0.0f ? 0.0f : acc / den;
      r *= sigmoidf_acc(gate_v[k]);
      p.output[out_index] = r;
    } else if (p.splits == 1) {
      write_final<kMD, G>(p, token, kvh, idx, den, acc);
    } else {
      store_through(&po[idx], acc);
      if (idx % kMD == 0) {
        store_through(&pml[g * 2 + 0], mx);
        store_through(&pml[g * 2 + 1], den);
      }
    }
  }
}

}  // namespace

hipError_t launch_decode_short(const DecodeParams& p, uint32_t group, dim3 grid,
                               hipStream_t stream) {
  const PrologueFold none{};
  switch (group) {
    case 1:
      attention_decode_short_kernel<1, false><<<grid, 64 * kSWaves, 0, stream>>>(p, none);
      break;
    case 2:
      attention_decode_short_kernel<2, false><<<grid, 64 * kSWaves, 0, stream>>>(p, none);
      break;
    case 4:
      attention_decode_short_kernel<4, false><<<grid, 64 * kSWaves, 0, stream>>>(p, none);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode_short_prologue(const DecodeParams& p, const PrologueFold& f,
                                        uint32_t group, hipStream_t stream) {
  if (p.tokens != 1 || p.splits != 1 || p.keys_per_split != p.start_position + 1u ||
      p.start_position >= p.capacity_tokens || p.heads != group * p.kv_heads) {
    return hipErrorInvalidValue;
  }
  const dim3 grid(1, p.kv_heads, 1);
  switch (group) {
    case 1:
      attention_decode_short_kernel<1, true><<<grid, 64 * kSWaves, 0, stream>>>(p, f);
      break;
    case 2:
      attention_decode_short_kernel<2, true><<<grid, 64 * kSWaves, 0, stream>>>(p, f);
      break;
    case 4:
      attention_decode_short_kernel<4, true><<<grid, 64 * kSWaves, 0, stream>>>(p, f);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace decode
}  // namespace kraken
