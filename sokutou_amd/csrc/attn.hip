// One-token GQA decode attention with fused per-head q/k RMSNorm, rotate-half RoPE and bf16 KV append.
//
// Replaces the reference's `attn` kernel (qwen3/kernels.py:338-414), which runs one 256-thread block per kv head
// (8 blocks on the whole GPU) and keeps every score of the cache in shared memory. Here the cache length is split:
// block (kvh, split) takes positions [t0, t1) of kv head kvh for both of its q heads and produces an
// unnormalised partial (running max m, sum l, o = Σ exp(s - m) v). The last block of a head to finish (an
// arrival counter per head in the workspace) merges the partials with a log-sum-exp combine and writes the
// output, so the whole step is one launch of nkv * nsplit blocks.
//
// Layout inside a block (4 wave64s): for the score and P·V passes lane (g = lane / 16, sl = lane % 16) of wave w
// reads dims [8 sl, 8 sl + 8) of position t0 + 16 i + 4 w + g; one 16-byte load covers the 8 bf16 values and a
// score is a 16-lane DPP row sum. Both q heads share each K and V load (GQA ratio 2).
//
// Numerics follow the reference: K is stored as bf16 (round to nearest even) after norm and RoPE and the
// rounded value is used for its own score; V is stored without normalisation; q stays fp32 and is scaled by
// 1/sqrt(128) after RoPE; softmax subtracts the max and uses expf; division happens once at the end.
#include "common.h"
#include "internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kSplitMax = 32;
constexpr int kPart = SK_HD + 2;  // m, l, o[128]
constexpr float kInvSqrtHd = 0.08838834764831845f;

int nsplit_for(int max_len) {
  int n = (max_len + 15) / 16;
  return n < 1 ? 1 : (n > kSplitMax ? kSplitMax : n);
}
int64_t part_bytes(int nkv, int nsplit) { return ((int64_t)nkv * 2 * nsplit * kPart * 4 + 255) / 256 * 256; }

template <int CT>
__device__ __forceinline__ void load8(const typename Cache<CT>::T* p, float* o) {
  if constexpr (CT == SK_CT_BF16) {
    uint4 v = *(const uint4*)p;
    o[0] = bf2f(v.x & 0xffffu); o[1] = bf2f(v.x >> 16); o[2] = bf2f(v.y & 0xffffu); o[3] = bf2f(v.y >> 16);
    o[4] = bf2f(v.z & 0xffffu); o[5] = bf2f(v.z >> 16); o[6] = bf2f(v.w & 0xffffu); o[7] = bf2f(v.w >> 16);
  } else {
    float4 a = *(const float4*)p, b = *(const float4*)(p + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
}

template <int CT>
__global__ __launch_bounds__(kThreads) void k_attn(const float* __restrict__ qkv, const float* __restrict__ qn,
                                                   const float* __restrict__ kn, float eps, const float* __restrict__ rope,
                                                   typename Cache<CT>::T* __restrict__ Kc,
                                                   typename Cache<CT>::T* __restrict__ Vc,
                                                   const int64_t* __restrict__ pos_ptr, int pos_add, int max_len, int nq,
                                                   int nkv, float* __restrict__ out, float* __restrict__ part,
                                                   unsigned* __restrict__ counters, int nsplit, int chunk_max) {
  using C = Cache<CT>;
  extern __shared__ float sc[];  // [2][chunk_max] scores, then probabilities
  __shared__ float qsh[2][SK_HD];
  __shared__ float ksh[SK_HD];
  __shared__ float vsh[SK_HD];
  __shared__ float red[8];
  __shared__ float opart[4][4][16][16];  // [wave][row g][sl][head*8 + i]
  __shared__ int is_last;
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int t = threadIdx.x, p = t >> 7, d = t & (SK_HD - 1), w = t >> 6, lane = t & 63, g = lane >> 4, sl = lane & 15;
  int pos = (pos_ptr ? (int)pos_ptr[0] : 0) + pos_add;
  const bool pos_ok = pos >= 0 && pos < max_len;
  if (!pos_ok) pos = 0;
  const int T = pos_ok ? pos + 1 : 0;
  const int chunk = (T + nsplit - 1) / nsplit;
  const int t0 = split * chunk, t1 = min(T, t0 + chunk);
  const int n = t1 > t0 ? t1 - t0 : 0;
  const bool has_pos = pos_ok && t0 <= pos && pos < t1;
  typename C::T* Kh = Kc + (size_t)kvh * max_len * SK_HD;
  typename C::T* Vh = Vc + (size_t)kvh * max_len * SK_HD;

  float m = -INFINITY, l = 0.f, o = 0.f;
  if (n > 0) {
    // ---- q of heads 2 kvh + p, and (for the block that owns pos) the new k / v -----------------------------
    const float c = rope[(size_t)pos * SK_HD + (d & 63)], s = rope[(size_t)pos * SK_HD + 64 + (d & 63)];
    const float qv = qkv[(2 * kvh + p) * SK_HD + d];
    const float kv = has_pos ? qkv[nq * SK_HD + p * nkv * SK_HD + kvh * SK_HD + d] : 0.f;
    float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
    if (lane == 0) { red[w] = sq; red[4 + w] = sk; }
    __syncthreads();
    qsh[p][d] = qv * rsqrtf((red[2 * p] + red[2 * p + 1]) / SK_HD + eps) * qn[d];
    if (has_pos) {
      if (p == 0) ksh[d] = kv * rsqrtf((red[4] + red[5]) / SK_HD + eps) * kn[d];
      else vsh[d] = C::rnd(kv);
    }
    __syncthreads();
    const float qr = (qsh[p][d] * c + (d < 64 ? -qsh[p][d + 64] : qsh[p][d - 64]) * s) * kInvSqrtHd;
    float kr = 0.f;
    if (has_pos && p == 0) kr = C::rnd(ksh[d] * c + (d < 64 ? -ksh[d + 64] : ksh[d - 64]) * s);
    __syncthreads();
    qsh[p][d] = qr;
    if (has_pos) {
      if (p == 0) { ksh[d] = kr; Kh[(size_t)pos * SK_HD + d] = C::st(kr); }
      else Vh[(size_t)pos * SK_HD + d] = C::st(vsh[d]);
    }
    __syncthreads();

    // ---- scores for both q heads over [t0, t1) ------------------------------------------------------------
    float q0[8], q1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) { q0[i] = qsh[0][8 * sl + i]; q1[i] = qsh[1][8 * sl + i]; }
    for (int base = 0; base < n; base += 16) {
      const int jj = base + 4 * w + g;
      float k8[8];
      if (jj < n && t0 + jj == pos) {
#pragma unroll
        for (int i = 0; i < 8; i++) k8[i] = ksh[8 * sl + i];
      } else if (jj < n) {
        load8<CT>(Kh + (size_t)(t0 + jj) * SK_HD + 8 * sl, k8);
      } else {
#pragma unroll
        for (int i = 0; i < 8; i++) k8[i] = 0.f;
      }
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int i = 0; i < 8; i++) { s0 = __builtin_fmaf(q0[i], k8[i], s0); s1 = __builtin_fmaf(q1[i], k8[i], s1); }
      s0 = row16_sum(s0);
      s1 = row16_sum(s1);
      if (sl == 0 && jj < n) { sc[jj] = s0; sc[chunk_max + jj] = s1; }
    }
    __syncthreads();

    // ---- local softmax statistics per head (threads 0-127: head 0, 128-255: head 1) ---------------------
    float* sp = sc + p * chunk_max;
    float mx = -INFINITY;
    for (int i = d; i < n; i += SK_HD) mx = fmaxf(mx, sp[i]);
    mx = wave_max(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    m = fmaxf(red[2 * p], red[2 * p + 1]);
    float sum = 0.f;
    for (int i = d; i < n; i += SK_HD) {
      const float e = expf(sp[i] - m);
      sp[i] = e;
      sum += e;
    }
    sum = wave_sum(sum);
    __syncthreads();
    if (lane == 0) red[4 + w] = sum;
    __syncthreads();
    l = red[4 + 2 * p] + red[4 + 2 * p + 1];

    // ---- o = Σ p_j V_j for both heads ---------------------------------------------------------------------
    float a0[8], a1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) { a0[i] = 0.f; a1[i] = 0.f; }
    for (int base = 0; base < n; base += 16) {
      const int jj = base + 4 * w + g;
      if (jj < n) {
        float v8[8];
        if (t0 + jj == pos) {
#pragma unroll
          for (int i = 0; i < 8; i++) v8[i] = vsh[8 * sl + i];
        } else {
          load8<CT>(Vh + (size_t)(t0 + jj) * SK_HD + 8 * sl, v8);
        }
        const float e0 = sc[jj], e1 = sc[chunk_max + jj];
#pragma unroll
        for (int i = 0; i < 8; i++) { a0[i] = __builtin_fmaf(e0, v8[i], a0[i]); a1[i] = __builtin_fmaf(e1, v8[i], a1[i]); }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) { opart[w][g][sl][i] = a0[i]; opart[w][g][sl][8 + i] = a1[i]; }
    __syncthreads();
    o = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ww++)
#pragma unroll
      for (int gg = 0; gg < 4; gg++) o += opart[ww][gg][d >> 3][p * 8 + (d & 7)];
  }

  // ---- publish the partial, then the last block of this head merges ----------------------------------------
  float* P = part + ((size_t)(kvh * 2 + p) * nsplit + split) * kPart;
  if (d == 0) { P[0] = m; P[1] = l; }
  P[2 + d] = o;
  __syncthreads();
  if (t == 0) {
    __threadfence();
    const unsigned prev = atomicAdd(&counters[kvh], 1u);
    is_last = prev == (unsigned)(nsplit - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __threadfence();
  const float* Ph = part + (size_t)(kvh * 2 + p) * nsplit * kPart;
  float M = -INFINITY;
  for (int c = 0; c < nsplit; c++) M = fmaxf(M, Ph[(size_t)c * kPart]);
  float L = 0.f, O = 0.f;
  for (int c = 0; c < nsplit; c++) {
    const float mc = Ph[(size_t)c * kPart];
    if (mc == -INFINITY) continue;
    const float f = expf(mc - M);
    L = __builtin_fmaf(f, Ph[(size_t)c * kPart + 1], L);
    O = __builtin_fmaf(f, Ph[(size_t)c * kPart + 2 + d], O);
  }
  out[(2 * kvh + p) * SK_HD + d] = L > 0.f ? O / L : 0.f;
  if (t == 0) __hip_atomic_store(&counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" int64_t sk_attn_workspace_size(int nq, int nkv, int max_len) {
  if (nkv <= 0 || max_len <= 0) return 0;
  (void)nq;
  return part_bytes(nkv, nsplit_for(max_len)) + (int64_t)nkv * 4;
}

extern "C" int sk_attn(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc,
                       void* Vc, const int64_t* pos_ptr, int pos_add, int max_len, int nq, int nkv, float* out,
                       void* workspace, int64_t workspace_bytes, int ct, void* stream) {
  if (!qkv || !qn || !kn || !rope || !Kc || !Vc || !out || !workspace)
    return sk_set_error(SK_EINVAL, "sk_attn: null pointer");
  if (nkv <= 0 || nq != 2 * nkv || max_len <= 0)
    return sk_set_error(SK_EINVAL, "sk_attn: needs nq == 2*nkv and max_len > 0 (head_dim 128)");
  if (ct != SK_CT_BF16 && ct != SK_CT_F32) return sk_set_error(SK_EINVAL, "sk_attn: bad cache type");
  if (!SK_ALIGNED16(Kc) || !SK_ALIGNED16(Vc)) return sk_set_error(SK_EINVAL, "sk_attn: caches must be 16-byte aligned");
  if (!SK_ALIGNED16(workspace)) return sk_set_error(SK_EINVAL, "sk_attn: workspace must be 16-byte aligned");
  if (workspace_bytes < sk_attn_workspace_size(nq, nkv, max_len))
    return sk_set_error(SK_EWORKSPACE, "sk_attn: workspace too small");
  const int nsplit = nsplit_for(max_len);
  const int chunk_max = (max_len + nsplit - 1) / nsplit;
  float* part = (float*)workspace;
  unsigned* counters = (unsigned*)((char*)workspace + part_bytes(nkv, nsplit));
  hipStream_t st = (hipStream_t)stream;
  dim3 grid(nkv, nsplit);
  const size_t smem = 2 * (size_t)chunk_max * sizeof(float);
  if (ct == SK_CT_BF16)
    hipLaunchKernelGGL((k_attn<SK_CT_BF16>), grid, dim3(kThreads), smem, st, qkv, qn, kn, eps, rope, (bf16_t*)Kc,
                       (bf16_t*)Vc, pos_ptr, pos_add, max_len, nq, nkv, out, part, counters, nsplit, chunk_max);
  else
    hipLaunchKernelGGL((k_attn<SK_CT_F32>), grid, dim3(kThreads), smem, st, qkv, qn, kn, eps, rope, (float*)Kc,
                       (float*)Vc, pos_ptr, pos_add, max_len, nq, nkv, out, part, counters, nsplit, chunk_max);
  return sk_check_launch(hipGetLastError(), "sk_attn");
}
