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
// One block of 1024 threads, 4 entries per thread. The top_k-th largest key is found by a radix select over the
// four bytes of the order key, most significant first: a 256-bin LDS histogram of the entries that match the
// digits chosen so far, then one wave scans the bins from the top to find the digit where the count reaches the
// rank still needed. Every entry whose key is at least that threshold (ties included) and that is not -inf competes
// with v - log(-log(u)), u from Philox4x32-10 with counter (index, draw lo, draw hi, 0x51) and key (seed lo, seed
// hi); the largest wins, the lowest index on ties. Afterwards the draw counter advances by one.
__global__ __launch_bounds__(kSampleThreads) void k_sample_draw(const float* __restrict__ logits, int V, float inv_temp,
                                                                int top_k, uint8_t* __restrict__ seen, float rep_pen,
                                                                const uint8_t* __restrict__ suppress,
                                                                int64_t* __restrict__ ngen, int min_new, int eos,
                                                                const uint64_t* __restrict__ seed,
                                                                uint64_t* __restrict__ counter, int64_t* __restrict__ out,
                                                                int talker, int64_t* __restrict__ id0,
                                                                int64_t* __restrict__ pos) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_need;
  __shared__ float best_v[kSampleThreads / SK_WAVE];
  __shared__ int best_i[kSampleThreads / SK_WAVE];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const bool block_eos = talker && ngen && ngen[0] < min_new;
  float l[kPer];
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int i = t + j * kSampleThreads;
    float v = -INFINITY;
    if (i < V) {
      v = logits[i];
      if (talker) {
        if (seen && seen[i]) v = v < 0.f ? v * rep_pen : v / rep_pen;
        if (suppress && suppress[i]) v = -INFINITY;
        if (block_eos && i == eos) v = -INFINITY;
      }
      v *= inv_temp;
    }
    l[j] = v;
  }
  uint32_t thr = 0;
  if (top_k > 0 && top_k < V) {
    if (t == 0) { s_prefix = 0; s_need = (uint32_t)top_k; }
    for (int pass = 0; pass < 4; pass++) {
      const int shift = 24 - 8 * pass;
      if (t < 256) hist[t] = 0;
      __syncthreads();
      const uint32_t prefix = s_prefix, need = s_need;
#pragma unroll
      for (int j = 0; j < kPer; j++) {
        const int i = t + j * kSampleThreads;
        if (i >= V) continue;
        const uint32_t k = order_key(l[j]);
        if (pass == 0 || ((k ^ prefix) >> (shift + 8)) == 0) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
      __syncthreads();
      if (w == 0) {
        // lane L holds bins 255 - 4L .. 252 - 4L (descending); inclusive scan of the counts over the lanes
        uint32_t c[4], sum = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) { c[q] = hist[255 - (4 * lane + q)]; sum += c[q]; }
        uint32_t inc = sum;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const uint32_t y = __shfl_up(inc, o);
          if (lane >= o) inc += y;
        }
        const uint32_t before = inc - sum;
        if (before < need && inc >= need) {
          uint32_t acc = before;
#pragma unroll
          for (int q = 0; q < 4; q++) {
            if (acc + c[q] >= need) {
              const uint32_t digit = 255u - (uint32_t)(4 * lane + q);
              s_prefix = prefix | (digit << shift);
              s_need = need - acc;
              break;
            }
            acc += c[q];
          }
        }
      }
      __syncthreads();
    }
    thr = s_prefix;
  }
  const uint64_t sd = seed[0], cnt = counter[0];
  float best = -INFINITY;
  int bi = 0x7fffffff;
#pragma unroll
  for (int j = 0; j < kPer; j++) {
    const int i = t + j * kSampleThreads;
    if (i >= V) continue;
    const float v = l[j];
    if (order_key(v) < thr || v == -INFINITY) continue;
    const float g = gumbel(v, (uint32_t)i, cnt, (uint32_t)sd, (uint32_t)(sd >> 32));
    if (g > best || (g == best && i < bi)) { best = g; bi = i; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o);
    const int oi = __shfl_xor(bi, o);
    if (ob > best || (ob == best && oi < bi)) { best = ob; bi = oi; }
  }
  if (lane == 0) { best_v[w] = best; best_i[w] = bi; }
  __syncthreads();
  if (t != 0) return;
  for (int q = 0; q < kSampleThreads / SK_WAVE; q++)
    if (best_v[q] > best || (best_v[q] == best && best_i[q] < bi)) { best = best_v[q]; bi = best_i[q]; }
  const int64_t id = bi == 0x7fffffff ? 0 : bi;
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
    hipLaunchKernelGGL(k_sample_draw, dim3(1), dim3(kSampleThreads), 0, (hipStream_t)stream, logits, V, inv_temp, top_k,
                       seen, rep_pen, suppress, ngen, min_new, eos, seed, counter, out, talker, id0, pos);
    return sk_check_launch(hipGetLastError(), "sk_sample");
  }
  hipLaunchKernelGGL(k_sample_greedy, dim3(1), dim3(kSampleThreads), 0, (hipStream_t)stream, logits, V, seen, rep_pen,
                     suppress, ngen, min_new, eos, out, talker, id0, pos);
  return sk_check_launch(hipGetLastError(), "sk_sample");
}
