// Small kernels of the talker step (final RMSNorm, embedding rows, greedy sampling) and the library's
// error/status plumbing.
#include <stdio.h>
#include <string.h>

#include "common.h"
#include "internal.h"

namespace {

thread_local char g_err[512] = "";

// ---- RMSNorm (qwen3/kernels.py:312-319) --------------------------------------------------------------------
constexpr int kNormThreads = 256;
__global__ __launch_bounds__(kNormThreads) void k_rmsnorm(const float* __restrict__ h, const float* __restrict__ nw,
                                                           float eps, float* __restrict__ out, int K) {
  __shared__ float red[kNormThreads / SK_WAVE];
  float ss = 0.f;
  for (int i = threadIdx.x; i < K; i += kNormThreads) { const float v = h[i]; ss += v * v; }
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / SK_WAVE; i++) tot += red[i];
  const float inv = rsqrtf(tot / K + eps);
  for (int i = threadIdx.x; i < K; i += kNormThreads) out[i] = h[i] * inv * nw[i];
}

// ---- embedding row (qwen3/kernels.py:321-326) --------------------------------------------------------------
template <int CT>
__global__ void k_embed(const typename Cache<CT>::T* __restrict__ table, const int64_t* __restrict__ idx,
                        float* __restrict__ out, int dim) {
  const int64_t r = idx[0];
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x)
    out[i] = Cache<CT>::ld(table[(size_t)r * dim + i]);
}

// ---- talker input: sum of G codebook rows + pad (qwen3/kernels.py:328-336) ----------------------------------
template <int CT>
__global__ void k_talker_in(const uint64_t* __restrict__ tabs, const int64_t* __restrict__ codes,
                            const typename Cache<CT>::T* __restrict__ pad, float* __restrict__ out, int dim, int G) {
  typedef typename Cache<CT>::T ct;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < dim; i += gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int g = 0; g < G; g++) s += Cache<CT>::ld(((const ct*)tabs[g])[(size_t)codes[g] * dim + i]);
    out[i] = s + Cache<CT>::ld(pad[i]);
  }
}

// ---- greedy sampling with the talker processor (qwen3/sampler.py:37-159, do_sample = 0) ---------------------
constexpr int kSampleThreads = 1024;
constexpr int kPer = SK_MAX_V / kSampleThreads;

// Order-preserving key: larger value wins, then the lower index (lowest-index tie-break of the reference).
__device__ __forceinline__ uint64_t pick_key(float v, int i) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)k << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
}

__global__ __launch_bounds__(kSampleThreads) void k_sample_greedy(const float* __restrict__ logits, int V,
                                                                  uint8_t* __restrict__ seen, float rep_pen,
                                                                  const uint8_t* __restrict__ suppress,
                                                                  int64_t* __restrict__ ngen, int min_new, int eos,
                                                                  int64_t* __restrict__ out, int talker,
                                                                  int64_t* __restrict__ id0, int64_t* __restrict__ pos) {
  __shared__ uint64_t best_w[kSampleThreads / SK_WAVE];
  const int t = threadIdx.x;
  const bool block_eos = talker && ngen && ngen[0] < min_new;
  uint64_t best = 0;  // key 0 is below every non-NaN value
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int i = t + j * kSampleThreads;
    if (i >= V) break;
    float v = logits[i];
    if (talker) {
      if (seen && seen[i]) v = v < 0.f ? v * rep_pen : v / rep_pen;
      if (suppress && suppress[i]) v = -INFINITY;
      if (block_eos && i == eos) v = -INFINITY;
    }
    if (v != v) continue;  // NaN never wins
    const uint64_t k = pick_key(v, i);
    best = k > best ? k : best;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t b = __shfl_xor(best, o);
    best = b > best ? b : best;
  }
  if ((t & 63) == 0) best_w[t >> 6] = best;
  __syncthreads();
  if (t != 0) return;
  for (int i = 1; i < kSampleThreads / SK_WAVE; i++) best = best_w[i] > best ? best_w[i] : best;
  best = best_w[0] > best ? best_w[0] : best;
  const int64_t id = best ? (int64_t)(0xffffffffu - (uint32_t)best) : 0;
  out[0] = id;
  if (talker) {
    if (id0) id0[0] = id;
    if (seen) seen[id] = 1;
    if (ngen) ngen[0] += 1;
    if (pos) pos[0] += 1;
  }
}

// ---- sampled pick: processor, temperature, top-k threshold, Gumbel-max (qwen3/sampler.py:37-159) -----------------
// One block of 1024 threads; thread t holds entries t + 1024 j (j < 4) in registers as processed values and their
// order keys. The threshold (the key of the top_k-th largest value, ties kept) is found without a histogram:
//  * bound: the top_k-th largest of 256 group maxima (16 consecutive entries per group, a DPP row max) is a lower
//    bound of the threshold, since the maxima are themselves entries (top_k <= 256);
//  * candidates: the keys at or above the bound are compacted into LDS (one ballot per register and one LDS atomic
//    per wave for the wave's offset); typically a few times top_k of them;
//  * wave 0 bisects the key space, bit by bit from the highest bit where the bound and the largest key differ,
//    counting the candidates at or above each probe with ballots. Below the bound every count reaches top_k, as it
//    does over all entries, so the result is the full-vocabulary threshold.
// Larger top_k (256 < top_k < V) bisects over all entries, every wave counting its own with ballots per step.
// Entries past V carry key 0, which no probe counts (every probe is at least 1). Then every entry at or above the
// threshold that is not -inf draws its Gumbel value v - log(-log(u)), u from Philox4x32-10 with counter (index,
// draw lo, draw hi, 0x51) and key (seed lo, seed hi); the largest wins, the lowest index on ties (a wave max of the
// value, then a wave max of the complemented index among the lanes holding it). Afterwards the draw counter advances.
constexpr int kDrawThreads = 1024, kDrawWaves = kDrawThreads / SK_WAVE, kDrawPer = SK_MAX_V / kDrawThreads;
constexpr int kBoundGroups = 256;  // groups of 16 entries: SK_MAX_V / 16

template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x124>(v));  // row_ror:4
  v = max(v, dpp_u32<0x128>(v));  // row_ror:8
  return v;
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {  // uniform result
  v = row16_max_u32(v);
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
// The largest key t in [lo, hi] whose count (keys >= t) reaches K, given count(lo) >= K: the bits above the highest
// bit where lo and hi differ are common to every such key; below it the key grows one bit at a time, each bit kept
// when the count at the key with that bit set still reaches K.
template <class F>
__device__ __forceinline__ uint32_t kth_key(uint32_t lo, uint32_t hi, uint32_t K, F count) {
  if (lo >= hi) return lo;
  const int top = 31 - __builtin_clz(lo ^ hi);
  uint32_t p = top == 31 ? 0u : lo & ~((2u << top) - 1u);
  for (int b = top; b >= 0; b--) {
    const uint32_t t = p | (1u << b);
    if (count(t) >= K) p = t;
  }
  return p;
}

__global__ __launch_bounds__(kDrawThreads) void k_sample_draw(const float* __restrict__ logits, int V, float inv_temp,
                                                               int top_k, uint8_t* __restrict__ seen, float rep_pen,
                                                               const uint8_t* __restrict__ suppress,
                                                               int64_t* __restrict__ ngen, int min_new, int eos,
                                                               const uint64_t* __restrict__ seed,
                                                               uint64_t* __restrict__ counter, int64_t* __restrict__ out,
                                                               int talker, int64_t* __restrict__ id0,
                                                               int64_t* __restrict__ pos) {
  __shared__ uint32_t gmax[kBoundGroups];
  __shared__ uint32_t cand[SK_MAX_V];
  __shared__ uint32_t wsum[kDrawWaves];
  __shared__ uint32_t wpick[kDrawWaves];
  __shared__ uint32_t s_n, s_lb, s_thr;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const bool block_eos = talker && ngen && ngen[0] < min_new;
  float xv[kDrawPer];
  uint32_t key[kDrawPer];
#pragma unroll
  for (int j = 0; j < kDrawPer; j++) {
    const int i = t + j * kDrawThreads;
    float v = -INFINITY;
    key[j] = 0u;
    if (i < V) {
      v = logits[i];
      if (talker) {
        if (seen && seen[i]) v = v < 0.f ? v * rep_pen : v / rep_pen;
        if (suppress && suppress[i]) v = -INFINITY;
        if (block_eos && i == eos) v = -INFINITY;
      }
      v *= inv_temp;
      key[j] = order_key(v);
    }
    xv[j] = v;
  }
  uint32_t thr = 0;  // 0 keeps every entry (top_k <= 0 or >= V)
  if (top_k > 0 && top_k < V) {
    const uint32_t K = (uint32_t)top_k;
    if (top_k <= kBoundGroups) {
      // bound: group maxima (lanes 16 r .. 16 r + 15 hold 16 consecutive entries of each j)
#pragma unroll
      for (int j = 0; j < kDrawPer; j++) {
        const uint32_t m = row16_max_u32(key[j]);
        if ((lane & 15) == 0) gmax[(j * kDrawWaves + w) * 4 + (lane >> 4)] = m;
      }
      if (t == 0) s_n = 0;
      __syncthreads();
      if (w == 0) {
        uint32_t g4[4], lo = 0xffffffffu, hi = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          g4[q] = gmax[lane + 64 * q];
          lo = min(lo, g4[q]);
          hi = max(hi, g4[q]);
        }
        lo = ~wave_max_u32(~lo);
        hi = wave_max_u32(hi);
        const uint32_t lb = kth_key(lo, hi, K, [&](uint32_t x) {
          uint32_t c = 0;
#pragma unroll
          for (int q = 0; q < 4; q++) c += (uint32_t)__popcll(__ballot(g4[q] >= x));
          return c;
        });
        if (lane == 0) s_lb = lb;
      }
      __syncthreads();
      const uint32_t lb = s_lb;
      // candidates: keys >= lb (key 0 is never a candidate: no probe counts it)
#pragma unroll
      for (int j = 0; j < kDrawPer; j++) {
        const bool take = key[j] >= lb && key[j] != 0u;
        const uint64_t msk = __ballot(take);
        uint32_t base = 0;
        if (lane == 0 && msk) base = atomicAdd(&s_n, (uint32_t)__popcll(msk));
        base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
        if (take) cand[base + __builtin_amdgcn_mbcnt_hi((uint32_t)(msk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)msk, 0u))] = key[j];
      }
      __syncthreads();
      if (w == 0) {
        const uint32_t n = s_n;
        uint32_t hi = 0;
        for (uint32_t c = (uint32_t)lane; c < n; c += 64) hi = max(hi, cand[c]);
        hi = wave_max_u32(hi);
        uint32_t r;
        if (n <= 256) {  // the candidate keys stay in registers for the whole bisection
          uint32_t c4[4];
#pragma unroll
          for (int q = 0; q < 4; q++) c4[q] = (uint32_t)(lane + 64 * q) < n ? cand[lane + 64 * q] : 0u;
          r = kth_key(lb, hi, K, [&](uint32_t x) {
            uint32_t c = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) c += (uint32_t)__popcll(__ballot(c4[q] >= x));
            return c;
          });
        } else {
          r = kth_key(lb, hi, K, [&](uint32_t x) {
            uint32_t c = 0;
            for (uint32_t b = 0; b < n; b += 64) {
              const uint32_t i = b + (uint32_t)lane;
              c += (uint32_t)__popcll(__ballot(i < n && cand[i] >= x));
            }
            return c;
          });
        }
        if (lane == 0) s_thr = r;
      }
      __syncthreads();
      thr = s_thr;
    } else {
      // every wave counts its own keys per probe; the counts meet in LDS (two barriers per bit)
      uint32_t p = 0;
      for (int b = 31; b >= 0; b--) {
        const uint32_t x = p | (1u << b);
        uint32_t c = 0;
#pragma unroll
        for (int j = 0; j < kDrawPer; j++) c += (uint32_t)__popcll(__ballot(key[j] >= x));
        if (lane == 0) wsum[w] = c;
        __syncthreads();
        uint32_t tot = 0;
#pragma unroll
        for (int q = 0; q < kDrawWaves; q++) tot += wsum[q];
        __syncthreads();
        if (tot >= K) p = x;
      }
      thr = p;
    }
  }
  // Gumbel-max over the kept entries
  const uint64_t sd = seed[0], cnt = counter[0];
  float best = -INFINITY;
  uint32_t bi = 0xffffffffu;
#pragma unroll
  for (int j = 0; j < kDrawPer; j++) {
    const int i = t + j * kDrawThreads;
    if (i >= V || key[j] < thr || xv[j] == -INFINITY) continue;
    const float g = gumbel(xv[j], (uint32_t)i, cnt, (uint32_t)sd, (uint32_t)(sd >> 32));
    if (g > best || (g == best && (uint32_t)i < bi)) { best = g; bi = (uint32_t)i; }  // NaN never wins
  }
  // wave: the largest value (as an order key; -0 made +0 so equal values have equal keys), then the lowest index
  // among the lanes holding it
  const uint32_t mk = order_key(best == 0.f ? 0.f : best);
  const uint32_t bk = wave_max_u32(mk);
  const uint32_t bidx = ~wave_max_u32(mk == bk ? ~bi : 0u);
  if (lane == 0) { wsum[w] = bk; wpick[w] = bidx; }
  __syncthreads();
  if (w != 0) return;
  const uint32_t k2 = lane < kDrawWaves ? wsum[lane] : 0u;
  const uint32_t i2 = lane < kDrawWaves ? wpick[lane] : 0xffffffffu;
  const uint32_t tk = wave_max_u32(k2);
  const uint32_t pick = ~wave_max_u32(k2 == tk ? ~i2 : 0u);
  if (lane != 0) return;
  const int64_t id = pick >= (uint32_t)V ? 0 : (int64_t)pick;  // nothing kept: index 0
  out[0] = id;
  counter[0] = cnt + 1;
  if (talker) {
    if (id0) id0[0] = id;
    if (seen) seen[id] = 1;
    if (ngen) ngen[0] += 1;
    if (pos) pos[0] += 1;
  }
}

}  // namespace

int sk_set_error(int rc, const char* msg) {
  snprintf(g_err, sizeof g_err, "%s", msg);
  return rc;
}

int sk_check_launch(hipError_t e, const char* where) {
  if (e == hipSuccess) return SK_OK;
  snprintf(g_err, sizeof g_err, "%s: %s", where, hipGetErrorString(e));
  return SK_ELAUNCH;
}

extern "C" const char* sk_version(void) { return "sokutou_amd 0.1.0 (gfx950)"; }
extern "C" const char* sk_last_error(void) { return g_err; }

extern "C" int sk_device_check(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return sk_set_error(SK_EDEVICE, "sk_device_check: no HIP device");
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) return sk_set_error(SK_EDEVICE, "sk_device_check: no properties");
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0) {
    snprintf(g_err, sizeof g_err, "sk_device_check: device is %s, this build targets gfx950", p.gcnArchName);
    return SK_EDEVICE;
  }
  return SK_OK;
}

extern "C" int sk_rmsnorm(const float* h, const float* nw, float eps, float* out, int K, void* stream) {
  if (!h || !nw || !out || K <= 0) return sk_set_error(SK_EINVAL, "sk_rmsnorm: bad arguments");
  hipLaunchKernelGGL(k_rmsnorm, dim3(1), dim3(kNormThreads), 0, (hipStream_t)stream, h, nw, eps, out, K);
  return sk_check_launch(hipGetLastError(), "sk_rmsnorm");
}

extern "C" int sk_embed(const void* table, const int64_t* idx, float* out, int dim, int ct, void* stream) {
  if (!table || !idx || !out || dim <= 0) return sk_set_error(SK_EINVAL, "sk_embed: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  const int blocks = (dim + 255) / 256 < 8 ? (dim + 255) / 256 : 8;
  if (ct == SK_CT_BF16)
    hipLaunchKernelGGL(k_embed<SK_CT_BF16>, dim3(blocks), dim3(256), 0, st, (const bf16_t*)table, idx, out, dim);
  else if (ct == SK_CT_F32)
    hipLaunchKernelGGL(k_embed<SK_CT_F32>, dim3(blocks), dim3(256), 0, st, (const float*)table, idx, out, dim);
  else
    return sk_set_error(SK_EINVAL, "sk_embed: bad element type");
  return sk_check_launch(hipGetLastError(), "sk_embed");
}

extern "C" int sk_talker_in(const uint64_t* tabs, const int64_t* codes, const void* pad, float* out, int dim, int G,
                            int ct, void* stream) {
  if (!tabs || !codes || !pad || !out || dim <= 0 || G <= 0) return sk_set_error(SK_EINVAL, "sk_talker_in: bad arguments");
  hipStream_t st = (hipStream_t)stream;
  const int blocks = (dim + 255) / 256 < 8 ? (dim + 255) / 256 : 8;
  if (ct == SK_CT_BF16)
    hipLaunchKernelGGL(k_talker_in<SK_CT_BF16>, dim3(blocks), dim3(256), 0, st, tabs, codes, (const bf16_t*)pad, out,
                       dim, G);
  else if (ct == SK_CT_F32)
    hipLaunchKernelGGL(k_talker_in<SK_CT_F32>, dim3(blocks), dim3(256), 0, st, tabs, codes, (const float*)pad, out, dim,
                       G);
  else
    return sk_set_error(SK_EINVAL, "sk_talker_in: bad element type");
  return sk_check_launch(hipGetLastError(), "sk_talker_in");
}

extern "C" int sk_sample(const float* logits, int V, float inv_temp, int top_k, int do_sample, uint8_t* seen,
                         float rep_pen, const uint8_t* suppress, int64_t* ngen, int min_new, int eos,
                         const uint64_t* seed, uint64_t* counter, int64_t* out, int talker, int64_t* id0, int64_t* pos,
                         void* stream) {
  if (!logits || !out || V <= 0 || V > SK_MAX_V) return sk_set_error(SK_EINVAL, "sk_sample: bad arguments (V <= 4096)");
  if (talker && !ngen) return sk_set_error(SK_EINVAL, "sk_sample: talker mode needs ngen");
  if (do_sample) {
    if (!seed || !counter) return sk_set_error(SK_EINVAL, "sk_sample: sampling needs the device seed and counter");
    if (!(inv_temp > 0.f) || inv_temp == INFINITY) return sk_set_error(SK_EINVAL, "sk_sample: temperature must be > 0");
    hipLaunchKernelGGL(k_sample_draw, dim3(1), dim3(kDrawThreads), 0, (hipStream_t)stream, logits, V, inv_temp, top_k,
                       seen, rep_pen, suppress, ngen, min_new, eos, seed, counter, out, talker, id0, pos);
    return sk_check_launch(hipGetLastError(), "sk_sample");
  }
  hipLaunchKernelGGL(k_sample_greedy, dim3(1), dim3(kSampleThreads), 0, (hipStream_t)stream, logits, V, seen, rep_pen,
                     suppress, ngen, min_new, eos, out, talker, id0, pos);
  return sk_check_launch(hipGetLastError(), "sk_sample");
}
