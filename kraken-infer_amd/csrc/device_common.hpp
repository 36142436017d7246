// Device-side helpers shared by the gfx950 kernels: 64-lane wave reductions
// built from DPP row operations and ds_swizzle, fp16 packing, fast exp2.
//
// Lane groups used below (wave64):
//   reduce8  : lanes sharing (lane >> 3), i.e. 8 consecutive lanes
//   reduce32 : lanes sharing (lane >> 5)
//   across8  : lanes sharing (lane & 7) but differing in bits 3..4 (the 4 groups
//              of 8 within one 32-lane half): lane ^ 8 via row_ror:8, then
//              lane ^ 16 via ds_swizzle.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kraken {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// DPP control codes (GCN3+/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppRowMirror = 0x140;      // lane i <-> 15-i within 16
constexpr int kDppRowRor4 = 0x124;        // lane i <- (i+4) mod 16 within 16 (rotate by 4)
constexpr int kDppRowRor8 = 0x128;        // lane i <-> i^8 within 16 (rotate by 8)
// ds_swizzle bit mode: and_mask=0x1F, xor_mask=0x10 -> lane ^ 16 within 32.
constexpr int kSwizzleXor16 = 0x401F;

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
    __builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, true));
}

__device__ __forceinline__ float swizzle_xor16(float x) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), kSwizzleXor16));
}

// gfx950 lane-half exchanges (VALU, no LDS crossbar).  With the same register
// as both operands, v_permlane32_swap returns the pair (lanes 0-31 broadcast to
// both halves, lanes 32-63 broadcast to both halves); v_permlane16_swap does
// the same for the 16-lane rows of each half.  Combining the pair gives every
// lane op(x[l], x[l ^ 32]) or op(x[l], x[l ^ 16]).
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over the 8 lanes of an aligned 8-lane group; result in all 8 lanes.
__device__ __forceinline__ float reduce8_sum(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  return x;
}

__device__ __forceinline__ float reduce8_max(float x) {
  x = fmaxf(x, dpp<kDppQuadXor1>(x));
  x = fmaxf(x, dpp<kDppQuadXor2>(x));
  x = fmaxf(x, dpp<kDppRowHalfMirror>(x));
  return x;
}

// Sum over an aligned 32-lane half; result in all 32 lanes.
__device__ __forceinline__ float reduce32_sum(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppRowHalfMirror>(x);
  x += dpp<kDppRowMirror>(x);
  x += swizzle_xor16(x);
  return x;
}

// Combine the four 8-lane groups of each 32-lane half lane-wise (lane bits 3 and
// 4): every lane ends with the sum over lanes {l, l^8, l^16, l^24}.
__device__ __forceinline__ float across8_sum(float x) {
  x += dpp<kDppRowRor8>(x);
  x += swizzle_xor16(x);
  return x;
}

__device__ __forceinline__ float across8_max(float x) {
  x = fmaxf(x, dpp<kDppRowRor8>(x));
  x = fmaxf(x, swizzle_xor16(x));
  return x;
}

// Wave-uniform combination of the two 32-lane halves of a value that is already
// uniform within each half.
__device__ __forceinline__ float halves_sum(float x) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32));
}

__device__ __forceinline__ float halves_max(float x) {
  return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 0)),
               __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 32)));
}

// Full 64-lane sum, result uniform.
__device__ __forceinline__ float wave_sum(float x) { return halves_sum(reduce32_sum(x)); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

// Split fp32 operands for fp16 MFMA.  A value x is held as hi = f16(x) and
// lo = f16((x - hi) 2^11), so x = hi + 2^-11 lo to about 2^-21 relative; hi
// products and lo products go to separate fp32 accumulators and the lo sum is
// scaled by 2^-11 at the end.  Below the smallest normal f16 (2^-14) hi is zero
// and the whole value goes into the scaled lo, at f16 precision (at most 2^-25
// absolute).  The 2^11 scale keeps lo a normal f16: the matrix core can flush
// f16 denormal operands, and an unscaled lo = f16(x - hi) is denormal for every
// |x| < 2^-3 (and an f16 denormal hi lost that way dropped up to 6e-5 of a
// value: 3.5e-4 errors after the GDN norm-gated epilogue).  Valid for |x| below
// the f16 range (65504).  tests/test_split_f16.py and
// tests/test_decode_split_emulation.py check these bounds with every f16
// denormal flushed.
constexpr float kLoScale = 2048.0f;        // 2^11
constexpr float kLoUnscale = 1.0f / 2048.0f;
constexpr float kF16MinNormal = 6.103515625e-05f;  // 2^-14

__device__ __forceinline__ void split_f16(float x, half_t& hi, half_t& lo) {
  hi = static_cast<half_t>(__builtin_fabsf(x) < kF16MinNormal ? 0.0f : x);
  lo = static_cast<half_t>((x - static_cast<float>(hi)) * kLoScale);
}

// Raw (unswizzled, stride 0) buffer resource over `bytes` bytes from `base`;
// word 3 = 0x00020000 is the gfx9-family data format for raw dword access.
// A load whose offset is at or past `bytes` returns zeros without a memory
// access.  Base and size must be wave-uniform (the resource lives in SGPRs).
// readfirstlane states the uniformity to the compiler, which otherwise may not
// prove it and wraps every load in a waterfall loop over lanes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_buffer_rsrc(const void* base,
                                                                  uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, 0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                           0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Transposing 8-byte LDS read (ds_read_b64_tr_b16, gfx950) of four 16-bit
// values.  Within each group of 16 lanes, result lane l' gets element e (e < 4)
// = the 16-bit value at (address supplied by lane 4e + l'/4 of the group) +
// (l' % 4); so if lane 4e + q points at row e, columns 4q..4q+3 of a 4 x 16
// block, lane l' receives column l' of that block (checked on the device).
__device__ __forceinline__ half4_t read_tr16(const half_t* lds_address) {
  return __builtin_bit_cast(half4_t,
                            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)lds_address));
}

// Buffer resource words (raw, stride 0) over `bytes` bytes from `base`, for the
// inline-asm copies below; base and size are made wave-uniform.
__device__ __forceinline__ i32x4_t rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  i32x4_t r;
  r[0] = (int)__builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = (int)(__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) & 0xFFFFu);
  r[2] = (int)__builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000;
  return r;
}

// One direct-to-LDS 16-byte-per-lane copy (buffer_load_dwordx4 ... lds, gfx950):
// lane l's 16 bytes land at the wave-uniform LDS address `lds` + 16 l; an offset
// at or past the resource's byte count writes zeros without a memory access.
// Issued as inline asm so that the compiler does not make every later LDS read
// wait for it (it cannot tell the copy's target from the LDS being read); the
// caller awaits completion with an explicit s_waitcnt vmcnt.  M0 is set in the
// same statement, with the one wait state the M0 -> LDS-DMA hazard needs.  A
// kernel using this must have no other M0 user (tests/test_isa_m0.py checks the ISA), so
// declaring the reserved register clobbered is safe there.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy16_to_lds(i32x4_t rsrc, uint32_t voffset, const half_t* lds) {
  const uint32_t m0 =
    __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// The same copy to a wave-uniform LDS byte address (no generic-to-LDS pointer
// conversion per copy).
__device__ __forceinline__ void copy16_to_lds_addr(i32x4_t rsrc, uint32_t voffset,
                                                   uint32_t lds_address) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_address);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// The same copy with the nontemporal hint, for data read once (a KV stream).
__device__ __forceinline__ void copy16_to_lds_nt(i32x4_t rsrc, uint32_t voffset,
                                                 const half_t* lds) {
  const uint32_t m0 =
    __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t*)lds);
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :
               : "s"(m0), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// 16-byte buffer load with the nontemporal hint (cache policy bit NT).
__device__ __forceinline__ u32x4_t buffer_load_nt_b128(__amdgpu_buffer_rsrc_t rsrc,
                                                       uint32_t offset) {
  return __builtin_bit_cast(u32x4_t,
                            __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)offset, 0, 2));
}

// A store written through the L2 to memory (device scope: a vector store with
// SC1), for results a later launch reads: they do not stay dirty in the L2 for
// the kernel's end-of-launch release to write back after the last wave, and
// the next launch, whose workgroups run on other XCDs, reads them from memory
// in either case.  Measured: the decode split partials (C1 at L=4096
// 10.37 -> 10.03 us per step) and the fp16 GEMM's f32 output (Q5_K
// 6144 x 1024 at 1024 tokens 34.7 -> 32.9 us).  Not a win everywhere: the
// flash kernel's 16 MB of f16 partials (P=7168 81.5 -> 86.9 us) and the GDN
// decode state (2.54 -> 2.82 us) keep plain stores.
__device__ __forceinline__ void store_through(float* at, float v) {
  __hip_atomic_store(at, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace kraken
