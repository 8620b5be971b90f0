// Device helpers shared by the gfx950 kernels of the talker decode step.
// Wave64 throughout: reductions use DPP row operations, never 32-lane shuffles.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define SK_HD 128          // head_dim (fixed by the model family; the reference asserts it, qwen3/kernels.py:457)
#define SK_WAVE 64

typedef uint16_t bf16_t;

// ---- weight formats (the `wd` names of _Lin) -------------------------------------------------------------
enum SkWd { SK_WD_I8ROW = 0, SK_WD_I8G32 = 1, SK_WD_BF16 = 2, SK_WD_F32 = 3 };
// ---- KV-cache / embedding element type ------------------------------------------------------------------
enum SkCt { SK_CT_BF16 = 0, SK_CT_F32 = 1 };

// ---- scalar conversions ----------------------------------------------------------------------------------
__device__ __forceinline__ float bf2f(uint32_t u16) { return __uint_as_float(u16 << 16); }
// fp32 -> bf16, round to nearest even, NaN -> 0x7fc0 (same rule as torch's conversion)
__device__ __forceinline__ bf16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (bf16_t)(u >> 16);
}
__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 x;
  __builtin_memcpy(&x, &h, 2);
  return (float)x;
}
template <int CT> struct Cache;
template <> struct Cache<SK_CT_BF16> {
  typedef bf16_t T;
  static __device__ __forceinline__ float ld(T v) { return bf2f(v); }
  static __device__ __forceinline__ T st(float f) { return f2bf(f); }
  static __device__ __forceinline__ float rnd(float f) { return bf2f(f2bf(f)); }
};
template <> struct Cache<SK_CT_F32> {
  typedef float T;
  static __device__ __forceinline__ float ld(T v) { return v; }
  static __device__ __forceinline__ T st(float f) { return f; }
  static __device__ __forceinline__ float rnd(float f) { return f; }
};

// ---- DPP wave reductions ---------------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}
// Sum within each row of 16 lanes; every lane of the row receives it.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x124>(v);  // row_ror:4
  v += dpp<0x128>(v);  // row_ror:8
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x124>(v));
  v = fmaxf(v, dpp<0x128>(v));
  return v;
}
// Full wave64 sum, returned uniform (via lane 63).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp<0x142, 0xA>(v);  // row_bcast:15
  v += dpp<0x143, 0xC>(v);  // row_bcast:31
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  // combine the four 16-lane rows through scalar reads of one lane per row
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// ---- 16-byte weight chunk dot products -------------------------------------------------------------------
// A 16-byte chunk holds 16 int8, 8 bf16 or 4 fp32 weights; xp points at the matching fp32 inputs.
__device__ __forceinline__ float dot_i8x16(uint4 v, const float* __restrict__ xp) {
  float a0 = 0.f, a1 = 0.f;
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    float4 x = *(const float4*)(xp + 4 * i);
    float t = (float)(int8_t)(w[i]) * x.x;
    t = __builtin_fmaf((float)(int8_t)(w[i] >> 8), x.y, t);
    t = __builtin_fmaf((float)(int8_t)(w[i] >> 16), x.z, t);
    t = __builtin_fmaf((float)(int8_t)(w[i] >> 24), x.w, t);
    if (i & 1) a1 += t; else a0 += t;
  }
  return a0 + a1;
}
__device__ __forceinline__ float dot_bf16x8(uint4 v, const float* __restrict__ xp) {
  float4 a = *(const float4*)xp, b = *(const float4*)(xp + 4);
  float t = bf2f(v.x & 0xffffu) * a.x;
  t = __builtin_fmaf(bf2f(v.x >> 16), a.y, t);
  t = __builtin_fmaf(bf2f(v.y & 0xffffu), a.z, t);
  t = __builtin_fmaf(bf2f(v.y >> 16), a.w, t);
  t = __builtin_fmaf(bf2f(v.z & 0xffffu), b.x, t);
  t = __builtin_fmaf(bf2f(v.z >> 16), b.y, t);
  t = __builtin_fmaf(bf2f(v.w & 0xffffu), b.z, t);
  t = __builtin_fmaf(bf2f(v.w >> 16), b.w, t);
  return t;
}
__device__ __forceinline__ float dot_f32x4(uint4 v, const float* __restrict__ xp) {
  float4 a = *(const float4*)xp;
  float t = __uint_as_float(v.x) * a.x;
  t = __builtin_fmaf(__uint_as_float(v.y), a.y, t);
  t = __builtin_fmaf(__uint_as_float(v.z), a.z, t);
  t = __builtin_fmaf(__uint_as_float(v.w), a.w, t);
  return t;
}

// Elements per 16-byte chunk for a weight format.
template <int WD> struct WdInfo;
template <> struct WdInfo<SK_WD_I8ROW> { static constexpr int E = 16, BYTES = 1; };
template <> struct WdInfo<SK_WD_I8G32> { static constexpr int E = 16, BYTES = 1; };
template <> struct WdInfo<SK_WD_BF16> { static constexpr int E = 8, BYTES = 2; };
template <> struct WdInfo<SK_WD_F32> { static constexpr int E = 4, BYTES = 4; };

// Dot of chunk c of row `row` (K elements) with xp; applies group scales for i8g32 inside.
template <int WD>
__device__ __forceinline__ float chunk_dot(uint4 v, const float* __restrict__ xp, const uint16_t* __restrict__ S,
                                           int row, int K, int c) {
  if constexpr (WD == SK_WD_I8ROW) return dot_i8x16(v, xp);
  else if constexpr (WD == SK_WD_I8G32) return h2f(S[(size_t)row * (K >> 5) + (c >> 1)]) * dot_i8x16(v, xp);
  else if constexpr (WD == SK_WD_BF16) return dot_bf16x8(v, xp);
  else return dot_f32x4(v, xp);
}
// Row-level scale applied after the dot (i8row only).
template <int WD>
__device__ __forceinline__ float row_scale(const uint16_t* __restrict__ S, int row) {
  if constexpr (WD == SK_WD_I8ROW) return bf2f(S[row]);
  else return 1.f;
}

// ---- address space and uniformity ----------------------------------------------------------------------------
// A pointer read from memory (a descriptor table) is generic to the compiler. Loads through it become FLAT
// instructions, which count against the LDS wait counter as well, so every later LDS wait would also wait for
// them; and a buffer resource built from it needs a waterfall loop. `gptr` views memory as global, `uniform`
// moves a wave-uniform pointer into scalar registers.
template <class T> using gptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ T* uniform(T* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (T*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
template <class T>
__device__ __forceinline__ T gload(const T* p) { return *(gptr<const T>)p; }
template <class T>
__device__ __forceinline__ void gstore(T* p, T v) { *(gptr<T>)p = v; }

// ---- streaming loads -------------------------------------------------------------------------------------
// Weights are read once per frame: nontemporal hint keeps them from displacing reused lines in L2/MALL.
__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  u32x4 r = __builtin_nontemporal_load((gptr<const u32x4>)p);
  return make_uint4(r.x, r.y, r.z, r.w);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.f + expf(-g)) * u; }

// ---- device-coherent scalar accesses (sc1: visible to every XCD without an L2 writeback/invalidate) -------
__device__ __forceinline__ float ld_dev(const float* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_dev(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ uint32_t ld_dev(const uint32_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void st_dev(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// ---- buffer accesses with an explicit cache policy ----------------------------------------------------------
// `base` must be uniform across the wave (it becomes the SGPR buffer resource); per-lane offsets are in bytes.
// kPolDev (sc1) makes a load or store coherent at device scope, across all XCDs, without any L2 writeback or
// invalidate instruction.
constexpr int kPolDev = 16;
constexpr int kPolStream = 2;  // nt
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, 0x7fffffff, 0x00020000);
}
template <int POL = kPolDev>
__device__ __forceinline__ float buf_ldf(const void* base, uint32_t off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(make_rsrc(base), off, 0, POL));
}
template <int POL = kPolDev>
__device__ __forceinline__ void buf_stf(void* base, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), make_rsrc(base), off, 0, POL);
}

// ---- sampled picks ---------------------------------------------------------------------------------------------
// Order-preserving key of an fp32 value (the sign bit set for positives, all bits flipped for negatives).
__device__ __forceinline__ uint32_t order_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);  // all bits flipped for negatives, the sign for the rest
}
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): ten rounds of two 32x32->64-bit products with the published
// multipliers, the high halves xored with the other counter words and the key, the key bumped by Weyl constants.
__device__ __forceinline__ uint4 philox4x32_10(uint4 c, uint32_t k0, uint32_t k1) {
#pragma unroll
  for (int r = 0; r < 10; r++) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c.x, p1 = (uint64_t)0xCD9E8D57u * c.z;
    c = make_uint4((uint32_t)(p1 >> 32) ^ c.y ^ k0, (uint32_t)p1, (uint32_t)(p0 >> 32) ^ c.w ^ k1, (uint32_t)p0);
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c;
}
// The Gumbel-perturbed value of entry i for draw `cnt` under key (k0, k1): v - log(-log(u)), u in (0, 1) from the
// top 24 bits of the first Philox word of counter (i, draw lo, draw hi, 0x51).
__device__ __forceinline__ float gumbel(float v, uint32_t i, uint64_t cnt, uint32_t k0, uint32_t k1) {
  const uint4 r = philox4x32_10(make_uint4(i, (uint32_t)cnt, (uint32_t)(cnt >> 32), 0x51u), k0, k1);
  const float u = ((float)(r.x >> 8) + 0.5f) * (1.0f / 16777216.0f);
  return v - logf(-logf(u));
}

