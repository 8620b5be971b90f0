// One-token GQA decode attention with fused per-head q/k RMSNorm, rotate-half RoPE and bf16 KV append.
//
// Replaces the reference's `attn` kernel (qwen3/kernels.py:338-414), which runs one 256-thread block per kv head
// (8 blocks on the whole GPU) and keeps every score of the cache in shared memory. Here the cache length is split:
// block (kvh, split) takes positions [t0, t1) of kv head kvh for both of its q heads and produces an
// unnormalised partial (max m, sum l, o = Σ exp(s - m) v). The last block of a head to arrive (a counter per head
// in the workspace) merges the partials with a log-sum-exp combine and writes the output, so the whole step is
// one launch of nkv * nsplit blocks.
//
// Decode attention moves few bytes per block, so its time is the number of dependent memory round trips. The
// kernel has three: the position together with the block's first 64 K/V rows (the split boundaries depend only on
// the cache length, so these loads need no position), then every input that depends on the position (q, the new
// k/v, the RoPE row, the norm weights), then publishing the partial, and one batch of partial loads in the merging
// block.
//
// Layout inside a block (4 wave64s): lane (g = lane / 16, sl = lane % 16) of wave w holds dims [8 sl, 8 sl + 8)
// of positions t0 + 16 i + 4 w + g (i = 0..3); one 16-byte load covers 8 bf16 values and a score is a 16-lane
// DPP row sum. Both q heads of the kv head share each K and V load.
//
// Numerics follow the reference: K is stored as bf16 (round to nearest even) after norm and RoPE, and the
// rounded value is used for its own score; V is stored as given; q stays fp32 and is scaled by 1/sqrt(128) after
// RoPE; softmax subtracts the max and uses expf; one division at the end.
#include "common.h"
#include "internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kSplitMax = 16;
constexpr int kPass = 64;         // positions one block holds in registers per pass
constexpr int kPart = SK_HD + 2;  // m, l, o[128]
constexpr float kInvSqrtHd = 0.08838834764831845f;

// Splits of the cache: one block per head up to 128 positions (no merge), else chunks of a fixed number of positions,
// a multiple of the 64-position pass: 64 up to 1024 positions, beyond that the fewest 64s that keep 16 splits or
// fewer. Fixed chunks (rather than the cache so far divided evenly) let a block load its first pass before it knows
// the position, and never leave a pass of one or two positions.
struct SplitPlan {
  int chunk, nsplit;
};
SplitPlan split_plan(int max_len) {
  if (max_len <= 128) return {max_len, 1};
  const int chunk = kPass * ((max_len + kPass * kSplitMax - 1) / (kPass * kSplitMax));
  return {chunk, (max_len + chunk - 1) / chunk};
}
int nsplit_for(int max_len) { return split_plan(max_len).nsplit; }
constexpr int64_t part_bytes(int nkv, int nsplit) { return ((int64_t)nkv * 2 * nsplit * kPart * 4 + 255) / 256 * 256; }
// Workspace: the error word (byte 0) and the per-head arrival counters (from byte 4) first, at a fixed place for
// any cache length, then the partials, so one workspace serves calls with different max_len (talker and code
// predictor) without a partial landing on a counter.
constexpr uint32_t kErrBadPos = 5;  // the position lies outside [0, max_len): nothing is read or written
constexpr int64_t counter_bytes(int nkv) { return ((int64_t)nkv * 4 + 4 + 255) / 256 * 256; }

// 8 consecutive cache elements as raw bits: one uint4 for bf16, two for f32
template <int CT> struct Row8;
template <> struct Row8<SK_CT_BF16> {
  uint4 a;
  __device__ __forceinline__ void load(const bf16_t* p) { a = *(const uint4*)p; }
  __device__ __forceinline__ void zero() { a = make_uint4(0, 0, 0, 0); }
  __device__ __forceinline__ void get(float* o) const {
    o[0] = bf2f(a.x & 0xffffu); o[1] = bf2f(a.x >> 16); o[2] = bf2f(a.y & 0xffffu); o[3] = bf2f(a.y >> 16);
    o[4] = bf2f(a.z & 0xffffu); o[5] = bf2f(a.z >> 16); o[6] = bf2f(a.w & 0xffffu); o[7] = bf2f(a.w >> 16);
  }
};
template <> struct Row8<SK_CT_F32> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) { a = *(const float4*)p; b = *(const float4*)(p + 4); }
  __device__ __forceinline__ void zero() { a = b = make_float4(0.f, 0.f, 0.f, 0.f); }
  __device__ __forceinline__ void get(float* o) const {
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
};

template <int CT>
__global__ __launch_bounds__(kThreads) void k_attn(const float* __restrict__ qkv, const float* __restrict__ qn,
                                                   const float* __restrict__ kn, float eps, const float* __restrict__ rope,
                                                   typename Cache<CT>::T* __restrict__ Kc,
                                                   typename Cache<CT>::T* __restrict__ Vc,
                                                   const int64_t* __restrict__ pos_ptr, int pos_add, int max_len, int nq,
                                                   int nkv, float* __restrict__ out, float* __restrict__ part,
                                                   unsigned* __restrict__ err, unsigned* __restrict__ counters,
                                                   int chunk, int nsplit) {
  using C = Cache<CT>;
  __shared__ float qsh[2][SK_HD];
  __shared__ float ksh[SK_HD];
  __shared__ float vsh[SK_HD];
  __shared__ float sc[2][kPass];
  __shared__ float opart[4][4][16][17];  // [wave][row g][sl][head*8 + i], padded against bank conflicts
  __shared__ float mls[2][kSplitMax][2];
  __shared__ int is_last;
  const int kvh = blockIdx.x, split = blockIdx.y;
  const int t = threadIdx.x, p = t >> 7, d = t & (SK_HD - 1), w = t >> 6, lane = t & 63, g = lane >> 4, sl = lane & 15;
  const int t0 = split * chunk;
  typename C::T* Kh = Kc + (size_t)kvh * max_len * SK_HD;
  typename C::T* Vh = Vc + (size_t)kvh * max_len * SK_HD;
  // the first pass's K/V rows, before the position: rows past the cache's end read its last row instead and, like
  // rows at or past the position, are never used (the row at the position comes from LDS)
  Row8<CT> kr8[4], vr8[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int row = min(t0 + 16 * i + 4 * w + g, max_len - 1);
    kr8[i].load(Kh + (size_t)row * SK_HD + 8 * sl);
    vr8[i].load(Vh + (size_t)row * SK_HD + 8 * sl);
  }
  const int64_t pos64 = (pos_ptr ? pos_ptr[0] : 0) + (int64_t)pos_add;
  if (pos64 < 0 || pos64 >= max_len) {
    // every block takes this exit (the position is uniform), so no counter moves and nothing is written
    if (kvh == 0 && split == 0 && t == 0) __hip_atomic_store(err, kErrBadPos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int pos = (int)pos64;
  const int T = pos + 1;
  const int t1 = min(T, t0 + chunk);
  const int n = t1 > t0 ? t1 - t0 : 0;
  const bool has_pos = t0 <= pos && pos < t1;

  float m = -INFINITY, l = 0.f, o = 0.f;  // running partial of head p, dim d
  for (int base = 0; base < n; base += kPass) {
    // ---- every load of the pass at once: K/V rows (later passes), then (first pass) q / new k,v / rope / norm
    if (base > 0) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int jj = base + 16 * i + 4 * w + g;
        if (jj < n && t0 + jj != pos) {
          kr8[i].load(Kh + (size_t)(t0 + jj) * SK_HD + 8 * sl);
          vr8[i].load(Vh + (size_t)(t0 + jj) * SK_HD + 8 * sl);
        } else {
          kr8[i].zero();
          vr8[i].zero();
        }
      }
    }
    if (base == 0) {
      // q of both heads, and in the block holding the position this step's k and v: one wave per vector (wave 0 q of
      // head 2 kvh, wave 1 q of head 2 kvh + 1, wave 2 k, wave 3 v), dims lane and lane + 64 per lane, so the per-head
      // RMSNorm is a wave sum and the rotate-half RoPE pair stays in the lane: one barrier
      if (w < 2 || has_pos) {
        const float* src = w < 2 ? qkv + (2 * kvh + w) * SK_HD : qkv + nq * SK_HD + (w - 2) * nkv * SK_HD + kvh * SK_HD;
        const float x0 = src[lane], x1 = src[lane + 64];
        if (w < 3) {
          const float* nw = w < 2 ? qn : kn;
          const float c = rope[(size_t)pos * SK_HD + lane], sn = rope[(size_t)pos * SK_HD + 64 + lane];
          const float inv = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / SK_HD + eps);
          const float y0 = x0 * inv * nw[lane], y1 = x1 * inv * nw[lane + 64];
          const float r0 = y0 * c + -y1 * sn, r1 = y1 * c + y0 * sn;
          if (w < 2) {
            qsh[w][lane] = r0 * kInvSqrtHd;
            qsh[w][lane + 64] = r1 * kInvSqrtHd;
          } else {
            const float k0 = C::rnd(r0), k1 = C::rnd(r1);
            ksh[lane] = k0;
            ksh[lane + 64] = k1;
            Kh[(size_t)pos * SK_HD + lane] = C::st(k0);
            Kh[(size_t)pos * SK_HD + lane + 64] = C::st(k1);
          }
        } else {
          const float v0 = C::rnd(x0), v1 = C::rnd(x1);
          vsh[lane] = v0;
          vsh[lane + 64] = v1;
          Vh[(size_t)pos * SK_HD + lane] = C::st(v0);
          Vh[(size_t)pos * SK_HD + lane + 64] = C::st(v1);
        }
      }
      __syncthreads();
    }
    // ---- scores of the pass for both q heads ---------------------------------------------------------------
    float q0[8], q1[8];
#pragma unroll
    for (int i = 0; i < 8; i++) { q0[i] = qsh[0][8 * sl + i]; q1[i] = qsh[1][8 * sl + i]; }
    const int np = min(kPass, n - base);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int jj = base + 16 * i + 4 * w + g;
      float k8[8];
      if (jj < n && t0 + jj == pos) {
#pragma unroll
        for (int e = 0; e < 8; e++) k8[e] = ksh[8 * sl + e];
      } else {
        kr8[i].get(k8);
      }
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) { s0 = __builtin_fmaf(q0[e], k8[e], s0); s1 = __builtin_fmaf(q1[e], k8[e], s1); }
      s0 = row16_sum(s0);
      s1 = row16_sum(s1);
      if (sl == 0 && jj - base < np) { sc[0][jj - base] = s0; sc[1][jj - base] = s1; }
    }
    __syncthreads();
    // ---- pass softmax statistics of both heads, computed by every wave from the pass's scores (no barrier) -----
    const float sv0 = lane < np ? sc[0][lane] : -INFINITY, sv1 = lane < np ? sc[1][lane] : -INFINITY;
    const float mp0 = wave_max(sv0), mp1 = wave_max(sv1);
    const float lp0 = wave_sum(lane < np ? expf(sv0 - mp0) : 0.f), lp1 = wave_sum(lane < np ? expf(sv1 - mp1) : 0.f);
    const float mp = p ? mp1 : mp0, lp = p ? lp1 : lp0;
    // ---- o_pass = Σ p_j V_j for both heads -------------------------------------------------------------------
    float a0[8], a1[8];
#pragma unroll
    for (int e = 0; e < 8; e++) { a0[e] = 0.f; a1[e] = 0.f; }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int jj = base + 16 * i + 4 * w + g;
      if (jj - base < np) {
        float v8[8];
        if (t0 + jj == pos) {
#pragma unroll
          for (int e = 0; e < 8; e++) v8[e] = vsh[8 * sl + e];
        } else {
          vr8[i].get(v8);
        }
        const float e0 = expf(sc[0][jj - base] - mp0), e1 = expf(sc[1][jj - base] - mp1);
#pragma unroll
        for (int e = 0; e < 8; e++) { a0[e] = __builtin_fmaf(e0, v8[e], a0[e]); a1[e] = __builtin_fmaf(e1, v8[e], a1[e]); }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) { opart[w][g][sl][e] = a0[e]; opart[w][g][sl][8 + e] = a1[e]; }
    __syncthreads();
    float op = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ww++)
#pragma unroll
      for (int gg = 0; gg < 4; gg++) op += opart[ww][gg][d >> 3][p * 8 + (d & 7)];
    // ---- fold the pass into the running partial --------------------------------------------------------------
    const float mn = fmaxf(m, mp);
    const float fo = m == -INFINITY ? 0.f : expf(m - mn), fp = expf(mp - mn);
    o = o * fo + op * fp;
    l = l * fo + lp * fp;
    m = mn;
    if (base + kPass < n) __syncthreads();  // sc / opart are rewritten by the next pass
  }

  if (nsplit == 1) {  // the whole cache in this block: no partial to merge
    out[(2 * kvh + p) * SK_HD + d] = l > 0.f ? o / l : 0.f;
    return;
  }
  // ---- publish the partial (device-coherent stores), count the arrival ---------------------------------------
  const uint32_t pofs = (uint32_t)((kvh * 2 + p) * nsplit + split) * kPart * 4;
  if (d == 0) { buf_stf(part, pofs, m); buf_stf(part, pofs + 4, l); }
  buf_stf(part, pofs + 8 + 4 * d, o);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&counters[kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = prev == (unsigned)(nsplit - 1);
  }
  __syncthreads();
  if (!is_last) return;
  // ---- merge: one batch of device-coherent loads, then the log-sum-exp combine --------------------------------
  if (t < 2 * nsplit) {
    const int pp = t / nsplit, cc = t % nsplit;
    const uint32_t of = (uint32_t)((kvh * 2 + pp) * nsplit + cc) * kPart * 4;
    mls[pp][cc][0] = buf_ldf(part, of);
    mls[pp][cc][1] = buf_ldf(part, of + 4);
  }
  float oc[kSplitMax];
#pragma unroll
  for (int cc = 0; cc < kSplitMax; cc++)
    oc[cc] = cc < nsplit ? buf_ldf(part, (uint32_t)((kvh * 2 + p) * nsplit + cc) * kPart * 4 + 8 + 4 * d) : 0.f;
  __syncthreads();
  float M = -INFINITY;
  for (int cc = 0; cc < nsplit; cc++) M = fmaxf(M, mls[p][cc][0]);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int cc = 0; cc < kSplitMax; cc++) {
    if (cc < nsplit && mls[p][cc][0] != -INFINITY) {
      const float f = expf(mls[p][cc][0] - M);
      L = __builtin_fmaf(f, mls[p][cc][1], L);
      O = __builtin_fmaf(f, oc[cc], O);
    }
  }
  out[(2 * kvh + p) * SK_HD + d] = L > 0.f ? O / L : 0.f;
  if (t == 0) __hip_atomic_store(&counters[kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

extern "C" int64_t sk_attn_workspace_size(int nq, int nkv, int max_len) {
  if (nkv <= 0 || max_len <= 0) return 0;
  (void)nq;
  return counter_bytes(nkv) + part_bytes(nkv, nsplit_for(max_len));
}

namespace {

// Checks shared by both entry points; SK_OK or the status already recorded.
int check_attn(const float* qkv, const float* qn, const float* kn, const float* rope, const void* Kc, const void* Vc,
               int max_len, int nq, int nkv, const float* out, int ct) {
  if (!qkv || !qn || !kn || !rope || !Kc || !Vc || !out) return sk_set_error(SK_EINVAL, "sk_attn: null pointer");
  if (nkv <= 0 || nq != 2 * nkv || max_len <= 0)
    return sk_set_error(SK_EINVAL, "sk_attn: needs nq == 2*nkv and max_len > 0 (head_dim 128)");
  if ((int64_t)nkv * 2 * kSplitMax * kPart * 4 >= (int64_t)1 << 31 || (int64_t)max_len * nkv * SK_HD * 4 >= (int64_t)1 << 40)
    return sk_set_error(SK_EINVAL, "sk_attn: sizes out of range");
  if (ct != SK_CT_BF16 && ct != SK_CT_F32) return sk_set_error(SK_EINVAL, "sk_attn: bad cache type");
  if (!SK_ALIGNED16(Kc) || !SK_ALIGNED16(Vc)) return sk_set_error(SK_EINVAL, "sk_attn: caches must be 16-byte aligned");
  return SK_OK;
}

int launch_attn(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc, void* Vc,
                const int64_t* pos_ptr, int pos_add, int max_len, int nq, int nkv, float* out, float* part,
                unsigned* err, unsigned* counters, int ct, hipStream_t st, const char* name) {
  const SplitPlan sp = split_plan(max_len);
  const int nsplit = sp.nsplit;
  dim3 grid(nkv, nsplit);
  if (ct == SK_CT_BF16)
    hipLaunchKernelGGL((k_attn<SK_CT_BF16>), grid, dim3(kThreads), 0, st, qkv, qn, kn, eps, rope, (bf16_t*)Kc,
                       (bf16_t*)Vc, pos_ptr, pos_add, max_len, nq, nkv, out, part, err, counters, sp.chunk, nsplit);
  else
    hipLaunchKernelGGL((k_attn<SK_CT_F32>), grid, dim3(kThreads), 0, st, qkv, qn, kn, eps, rope, (float*)Kc,
                       (float*)Vc, pos_ptr, pos_add, max_len, nq, nkv, out, part, err, counters, sp.chunk, nsplit);
  return sk_check_launch(hipGetLastError(), name);
}

}  // namespace

extern "C" int sk_attn(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc,
                       void* Vc, const int64_t* pos_ptr, int pos_add, int max_len, int nq, int nkv, float* out,
                       void* workspace, int64_t workspace_bytes, int ct, void* stream) {
  const int rc = check_attn(qkv, qn, kn, rope, Kc, Vc, max_len, nq, nkv, out, ct);
  if (rc != SK_OK) return rc;
  if (!workspace) return sk_set_error(SK_EINVAL, "sk_attn: null pointer");
  if (!SK_ALIGNED16(workspace)) return sk_set_error(SK_EINVAL, "sk_attn: workspace must be 16-byte aligned");
  if (workspace_bytes < sk_attn_workspace_size(nq, nkv, max_len))
    return sk_set_error(SK_EWORKSPACE, "sk_attn: workspace too small");
  unsigned* err = (unsigned*)workspace;
  float* part = (float*)((char*)workspace + counter_bytes(nkv));
  return launch_attn(qkv, qn, kn, eps, rope, Kc, Vc, pos_ptr, pos_add, max_len, nq, nkv, out, part, err, err + 1, ct,
                     (hipStream_t)stream, "sk_attn");
}

// ---- allocation-free variant -------------------------------------------------------------------------------------
// sk_attn_noalloc keeps its split-K scratch (error word, arrival counters, partials) in this file-scope device array
// instead of a caller workspace: at most kNoAllocMaxKv kv heads. Each device holds its own copy until the process
// ends. The host never passes the array's name to a kernel: the first call on a device looks up the device address
// with hipGetSymbolAddress and keeps it per device.
namespace {
constexpr int kNoAllocMaxKv = 16;
constexpr int64_t kNoAllocBytes = counter_bytes(kNoAllocMaxKv) + part_bytes(kNoAllocMaxKv, kSplitMax);
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

namespace {

void* g_scratch[kMaxDevices];  // device address of `scratch` per device (null until the first call there)

// Clears the error word and the arrival counters (the first counter_bytes of the scratch): a fill kernel, not a
// memset node, so the clear is also safe inside a captured graph.
__global__ void k_clear_words(unsigned* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace

extern "C" int sk_attn_noalloc(const float* qkv, const float* qn, const float* kn, float eps, const float* rope,
                               void* Kc, void* Vc, const int64_t* pos_ptr, int pos_add, int max_len, int nq, int nkv,
                               float* out, int* err, int ct, void* stream) {
  const int rc = check_attn(qkv, qn, kn, rope, Kc, Vc, max_len, nq, nkv, out, ct);
  if (rc != SK_OK) return rc;
  if (nkv > kNoAllocMaxKv)
    return sk_set_error(SK_EINVAL, "sk_attn_noalloc: at most 16 kv heads (the static scratch holds 260 KiB)");
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return sk_set_error(SK_EDEVICE, "sk_attn_noalloc: no current HIP device");
  hipStream_t st = (hipStream_t)stream;
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) return sk_check_launch(e != hipSuccess ? e : hipErrorInvalidSymbol,
                                                      "sk_attn_noalloc: hipGetSymbolAddress(scratch)");
    const int words = (int)(counter_bytes(kNoAllocMaxKv) / 4);
    hipLaunchKernelGGL(k_clear_words, dim3(1), dim3(words), 0, st, (unsigned*)p, words);
    const int lrc = sk_check_launch(hipGetLastError(), "sk_attn_noalloc: clearing the scratch counters");
    if (lrc != SK_OK) return lrc;
    g_scratch[dev] = p;
  }
  unsigned* base = (unsigned*)g_scratch[dev];
  float* part = (float*)((char*)base + counter_bytes(kNoAllocMaxKv));
  unsigned* errw = err ? (unsigned*)err : base;  // word 0 of the scratch when the caller takes no error word
  return launch_attn(qkv, qn, kn, eps, rope, Kc, Vc, pos_ptr, pos_add, max_len, nq, nkv, out, part, errw, base + 1, ct,
                     st, "sk_attn_noalloc");
}
