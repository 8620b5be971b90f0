// Batched talker decode: up to 16 streams per step, the projections as M=16 skinny GEMMs on the matrix cores.
//
// The reference decodes one stream (qwen3/fast.py:146 asserts batch 1) with M=1 GEMVs (qwen3/kernels.py:143-310).
// With 16 streams the projections are dense [16 x K] x [K x N] contractions, so they go to
// v_mfma_f32_16x16x32_bf16: int8 weights are exact in bf16 (|q| <= 127 has 7 significant bits), and each
// activation is split into kTerms bf16 terms (x = t0 + t1 + ..., t_i = bf16 of what the earlier terms left), so
// the products are exact and the sum keeps fp32 input precision; one bf16 term alone loses ~1e-2 of relative
// accuracy over 28 layers.
//
// Data layout (all activations have 16 rows; rows of inactive streams stay zero):
//   * weights: int8 in 1 KiB tiles. Tile (g, c) holds rows 16g..16g+15, columns 64c..64c+63; lane L = n + 16 j of
//     a wave reads bytes [16 L, 16 L + 16) = W[16 g + n][64 c + 16 j .. + 16] with one 16-byte load, so a wave's
//     load is one contiguous KiB. Within a chunk the contraction index is permuted identically for both operands
//     (MFMA h = 0, 1 of the chunk takes bytes 8h..8h+7 of every lane), which leaves the dot product unchanged.
//   * GEMM inputs: bf16 planes [kTerms][16][K]; lane (m + 16 j) reads x[m][64 c + 16 j .. + 16] of every plane.
//   * RMSNorm: the kernel that updates the residual h also writes the planes of bf16(h ⊙ w_next) and, per
//     16-column tile, the partial sums of squares of h; the consuming GEMM adds the partials of its row in a fixed
//     order and applies rsqrt(Σh²/K + eps) after the dot product (qwen3/kernels.py:180-186, 224).
//
// Per layer: qkv GEMM -> ragged split-K attention -> o GEMM (+= h, norm planes) -> gate/up GEMM (SwiGLU planes)
// -> down GEMM (+= h, norm planes of the next layer). Then the head GEMM and a greedy pick that also embeds the
// chosen token for the next step. Every kernel is deterministic: fixed reduction orders, no float atomics.
#include "common.h"
#include "internal.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

constexpr int kM = 16;         // rows of every activation buffer (streams)
#ifndef SK_BATCH_TERMS
#define SK_BATCH_TERMS 3
#endif
constexpr int kTerms = SK_BATCH_TERMS;
constexpr int kThreads = 256;
constexpr int kOutF32 = 0, kOutSwiglu = 1, kOutAcc = 2;
constexpr int kMaxSlices = 16;  // K slices of one GEMM (the plan keeps S = K / (64 CW) at or below this)

// ---- conversions ----------------------------------------------------------------------------------------------
// two floats whose low 16 bits are zero (small integers) -> packed bf16 pair, lo in the low half
__device__ __forceinline__ uint32_t pack_hi16(float lo, float hi) {
  return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
// 8 int8 (two dwords) -> 8 bf16, exactly
__device__ __forceinline__ bf16x8 i8x8_bf16(uint32_t a, uint32_t b) {
  u32x4 r;
  r.x = pack_hi16((float)(int8_t)a, (float)(int8_t)(a >> 8));
  r.y = pack_hi16((float)(int8_t)(a >> 16), (float)(int8_t)(a >> 24));
  r.z = pack_hi16((float)(int8_t)b, (float)(int8_t)(b >> 8));
  r.w = pack_hi16((float)(int8_t)(b >> 16), (float)(int8_t)(b >> 24));
  return __builtin_bit_cast(bf16x8, r);
}
__device__ __forceinline__ uint4 gload4(const uint4* p) {
  const u32x4 v = *(gptr<const u32x4>)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) {
  u32x4 r = {v.x, v.y, v.z, v.w};
  return __builtin_bit_cast(bf16x8, r);
}
// v as kTerms bf16 terms written to planes [kTerms][plane] at index i
__device__ __forceinline__ void store_terms(bf16_t* __restrict__ planes, size_t plane, size_t i, float v) {
#pragma unroll
  for (int t = 0; t < kTerms; t++) {
    const bf16_t b = f2bf(v);
    planes[t * plane + i] = b;
    v -= bf2f(b);
  }
}

struct GemmArgs {
  const bf16_t* x;      // input planes [kTerms][16][K]
  const float* ssp;     // [np][16] partial sums of squares behind x (NULL: no RMSNorm scale)
  int np;
  float eps;
  const uint8_t* w;     // tiled int8 weights
  const uint16_t* s;    // [N] bf16 row scales
  int N, K;
  float* out;           // F32: [16][N]; ACC: residual [16][N], updated in place
  bf16_t* act;          // SWIGLU: planes [kTerms][16][N/2]
  bf16_t* xn;           // ACC: planes [kTerms][16][N] of bf16(h ⊙ nw)
  const float* nw;      // ACC: next RMSNorm weight [N]
  float* ssp_out;       // ACC: [N/16][16] partial sums of squares of the updated residual
  int S;                // K slices (workgroups per row block)
  float* part;          // S > 1: [S][N / 16][256] partial sums
  unsigned* counters;   // S > 1: [row blocks] arrivals, zero between launches
};

// Workgroup (nb, slice) computes output row groups 4 R nb .. 4 R nb + 4 R - 1 (16 rows each; wave w owns R of them)
// for all 16 streams over K slice `slice` (CW chunks of 64). The slice's activation planes are read from memory once
// per workgroup into LDS and shared by the four waves, which split the rows: the planes' traffic is then one read
// per 64 R output rows instead of one per 16 R (when the waves split K instead, each workgroup read its whole slice
// for 16 R rows, and the planes of a step were read 2-3 times more often than the weights). Every load goes out at
// the top: the activation slice first (it is needed first), then the wave's weights (its HBM traffic). With S > 1
// slices the workgroups of a row block publish their sums (device-coherent stores) and the last to arrive adds them in
// slice order and runs the epilogue, so the result does not depend on arrival order.
template <int OUT, int R, int CW>
__global__ __launch_bounds__(kThreads) void k_bgemm(GemmArgs p) {
  constexpr int kSeg = kTerms * kM * CW * 8;            // 16-byte activation segments of the slice
  constexpr int kAct = (kSeg + kThreads - 1) / kThreads;  // per thread
  __shared__ uint4 xs[kTerms][CW][2][64];  // [term][chunk][half][lane m + 16 j]: bf16 x[m][64 c + 16 j + 8 h ..+8]
  __shared__ float ssq[16][kM];
  __shared__ float inv_s[kM];
  __shared__ int last_s;
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  const int C = p.K / 64;                 // 64-wide chunks per row
  const int G = p.N / 16;                 // row groups
  const int nb = blockIdx.x, slice = blockIdx.y;
  const int c0 = slice * CW;
  const int g0 = (nb * 4 + wv) * R;       // this wave's first row group
  const size_t plane = (size_t)kM * p.K;
  // the slice's activation segments: segment a = (t, m, q) holds bf16 x_t[m][64 c0 + 8 q .. + 8]
  uint4 av[kAct];
#pragma unroll
  for (int i = 0; i < kAct; i++) {
    const int a = tid + kThreads * i;
    if (a < kSeg) {
      const int t = a / (kM * CW * 8), m = (a / (CW * 8)) % kM, q = a % (CW * 8);
      av[i] = gload4((const uint4*)(p.x + t * plane + (size_t)m * p.K + (size_t)c0 * 64 + 8 * q));
    }
  }
  uint4 wq[CW][R];
#pragma unroll
  for (int c = 0; c < CW; c++)
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int g = min(g0 + r, G - 1);  // a row group past the matrix loads the last one (never stored)
      wq[c][r] = ld_stream((const uint4*)p.w + ((size_t)g * C + c0 + c) * 64 + lane);
    }
  float ssv = 0.f;  // this thread's share of the RMSNorm partial sums
  if (p.ssp)
    for (int q = tid >> 4; q < p.np; q += 16) ssv += gload(p.ssp + q * kM + (tid & 15));
#pragma unroll
  for (int i = 0; i < kAct; i++) {
    const int a = tid + kThreads * i;
    if (a < kSeg) {
      const int t = a / (kM * CW * 8), m = (a / (CW * 8)) % kM, q = a % (CW * 8);
      xs[t][q >> 3][q & 1][m + 16 * ((q >> 1) & 3)] = av[i];
    }
  }
  if (p.ssp) ssq[tid >> 4][tid & 15] = ssv;
  __syncthreads();
  if (p.ssp && tid < kM) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 16; q++) s += ssq[q][tid];
    inv_s[tid] = rsqrtf(s / p.K + p.eps);
  }
  f32x4 acc[R], acc2[R];  // first term, later terms (kept apart: the small terms accumulate at their own scale)
#pragma unroll
  for (int r = 0; r < R; r++) { acc[r] = f32x4{0.f, 0.f, 0.f, 0.f}; acc2[r] = acc[r]; }
#pragma unroll
  for (int c = 0; c < CW; c++) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      bf16x8 xa[kTerms];
#pragma unroll
      for (int t = 0; t < kTerms; t++) xa[t] = as_bf16x8(xs[t][c][h][lane]);
#pragma unroll
      for (int r = 0; r < R; r++) {
        const uint4 q = wq[c][r];
        const bf16x8 b = h ? i8x8_bf16(q.z, q.w) : i8x8_bf16(q.x, q.y);
        acc[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[0], b, acc[r], 0, 0, 0);
#pragma unroll
        for (int t = 1; t < kTerms; t++) acc2[r] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[t], b, acc2[r], 0, 0, 0);
      }
    }
  }
  // D[m][n] sits in lane n + 16 (m / 4), element m % 4
  float v[R][4];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int i = 0; i < 4; i++) v[r][i] = acc[r][i] + acc2[r][i];
  if (p.S > 1) {
    // partial of (slice, row group g): 256 floats, element i of lane L at 64 i + L
    const uint32_t stride = (uint32_t)G * 256u;
#pragma unroll
    for (int r = 0; r < R; r++)
      if (g0 + r < G)
#pragma unroll
        for (int i = 0; i < 4; i++)
          buf_stf(p.part, ((uint32_t)slice * stride + (uint32_t)(g0 + r) * 256u + 64u * i + lane) * 4u, v[r][i]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const unsigned prev = __hip_atomic_fetch_add(&p.counters[nb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last_s = prev == (unsigned)(p.S - 1);
    }
    __syncthreads();
    if (!last_s) return;
    // every slice's partial at once (one round trip), then the sum in slice order
    float pv[kMaxSlices][R][4];
#pragma unroll
    for (int q = 0; q < kMaxSlices; q++)
      if (q < p.S)
#pragma unroll
        for (int r = 0; r < R; r++)
#pragma unroll
          for (int i = 0; i < 4; i++)
            pv[q][r][i] = buf_ldf(p.part, ((uint32_t)q * stride + (uint32_t)min(g0 + r, G - 1) * 256u + 64u * i + lane) * 4u);
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float a = 0.f;
#pragma unroll
        for (int q = 0; q < kMaxSlices; q++)
          if (q < p.S) a += pv[q][r][i];
        v[r][i] = a;
      }
    if (tid == 0) __hip_atomic_store(&p.counters[nb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  } else {
    __syncthreads();  // inv_s
  }
  const int nl = lane & 15;
#pragma unroll
  for (int r = 0; r < R; r++) {
    if (g0 + r >= G) break;
    const int n = (g0 + r) * 16 + nl;
    const float sc = bf2f(p.s[n]);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = 4 * (lane >> 4) + i;
      const float y = v[r][i] * sc * (p.ssp ? inv_s[m] : 1.f);
      if constexpr (OUT == kOutF32) {
        p.out[(size_t)m * p.N + n] = y;
      } else if constexpr (OUT == kOutSwiglu) {
        const float u = dpp<0xB1>(y);  // lane L ^ 1: the up row next to this gate row
        if (!(nl & 1)) store_terms(p.act, (size_t)kM * (p.N / 2), (size_t)m * (p.N / 2) + n / 2, silu_mul(y, u));
      } else {
        float* hp = p.out + (size_t)m * p.N + n;
        const float hn = *hp + y;
        *hp = hn;
        store_terms(p.xn, (size_t)kM * p.N, (size_t)m * p.N + n, hn * p.nw[n]);
        const float ss = row16_sum(hn * hn);
        if (nl == 0) p.ssp_out[(g0 + r) * kM + m] = ss;
      }
    }
  }
}

// ---- weight tiling -----------------------------------------------------------------------------------------
__global__ void k_tile(const int8_t* __restrict__ w, int8_t* __restrict__ tiled, int N, int K) {
  // one thread per 16-byte lane slot: tile t = g * C + c, lane L = n + 16 j
  const size_t slot = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int C = K / 64;
  if (slot >= (size_t)N * K / 16) return;
  const int L = (int)(slot & 63);
  const size_t t = slot >> 6;
  const int g = (int)(t / C), c = (int)(t % C);
  const int n = L & 15, j = L >> 4;
  const uint4 v = *(const uint4*)(w + (size_t)(16 * g + n) * K + 64 * c + 16 * j);
  *(uint4*)(tiled + slot * 16) = v;
}

// ---- ragged split-K decode attention -----------------------------------------------------------------------
// Block (stream b, kv head g, split s) covers positions [128 s, 128 s + 128) of stream b's cache up to its current
// position, in two passes of 64 positions whose K/V rows are all loaded at the top; the split that holds the position
// also normalises, rotates and appends this step's K and V. Partials (max, sum, Σ p v) go to the workspace and a
// second launch (k_bmerge, one block per (b, g)) merges them in split order and writes the attention output as bf16
// term planes; a stream whose cache fits one split writes its output directly. The partials need no
// device-coherent stores and no arrival counter this way (the launch boundary orders them): 22.5 against 22.9 us
// per layer for merging in the attention launch by the last split to arrive. Numerics as sk_attn
// (qwen3/kernels.py:338-414).
constexpr int kPass = 64;
constexpr int kAttnPasses = 2;
constexpr int kAttnChunk = kPass * kAttnPasses;
constexpr int kAttnSplitMax = 32;  // max_len <= 4096
constexpr int kPart = SK_HD + 2;
constexpr float kInvSqrtHd = 0.08838834764831845f;

struct AttnArgs {
  const float* qkv;     // [16][(nq + 2 nkv) * 128]
  const float* qn;
  const float* kn;
  float eps;
  const float* rope;    // [max_len][cos 64 | sin 64]
  bf16_t* Kc;           // [batch][nkv][max_len][128]
  bf16_t* Vc;
  const int64_t* pos;   // [batch]
  int max_len, nq, nkv;
  bf16_t* att;          // planes [kTerms][16][nq * 128]
  float* part;          // [batch * nkv][2][kAttnSplitMax][kPart]
  int* err;
};

__device__ __forceinline__ void unpack8(uint4 v, float* o) {
  o[0] = bf2f(v.x & 0xffffu); o[1] = bf2f(v.x >> 16); o[2] = bf2f(v.y & 0xffffu); o[3] = bf2f(v.y >> 16);
  o[4] = bf2f(v.z & 0xffffu); o[5] = bf2f(v.z >> 16); o[6] = bf2f(v.w & 0xffffu); o[7] = bf2f(v.w >> 16);
}

__global__ __launch_bounds__(kThreads) void k_battn(AttnArgs a) {
  __shared__ float qsh[2][SK_HD];
  __shared__ float ksh[SK_HD];
  __shared__ float vsh[SK_HD];
  __shared__ float sc[2][kPass];
  __shared__ float red[16];
  __shared__ float opart[4][4][16][17];
  const int bg = blockIdx.x, b = bg / a.nkv, kvh = bg % a.nkv, split = blockIdx.y;
  const int t = threadIdx.x, p = t >> 7, d = t & (SK_HD - 1), w = t >> 6, lane = t & 63, gq = lane >> 4, sl = lane & 15;
  const int qs = (a.nq + 2 * a.nkv) * SK_HD;
  const int64_t pos64 = a.pos[b];
  const size_t ap = (size_t)kM * a.nq * SK_HD;
  if (pos64 < 0 || pos64 >= a.max_len) {  // a stream past its cache: zero output, error word set
    if (split == 0) {
      store_terms(a.att, ap, (size_t)b * a.nq * SK_HD + (2 * kvh + p) * SK_HD + d, 0.f);
      if (t == 0) atomicCAS(a.err, 0, 5);
    }
    return;
  }
  const int pos = (int)pos64, T = pos + 1, ns = (T + kAttnChunk - 1) / kAttnChunk;
  if (split >= ns) return;
  const int t0 = split * kAttnChunk, n = min(kAttnChunk, T - t0), npass = (n + kPass - 1) / kPass;
  const bool has_pos = split == ns - 1;
  bf16_t* Kh = a.Kc + ((size_t)b * a.nkv + kvh) * a.max_len * SK_HD;
  bf16_t* Vh = a.Vc + ((size_t)b * a.nkv + kvh) * a.max_len * SK_HD;
  const float* qrow = a.qkv + (size_t)b * qs;
  // lane (w, gq, sl) holds dims [8 sl, 8 sl + 8) of positions 16 i + 4 w + gq of a pass. Every load is issued
  // unconditionally (rows past the block's range read row t0 instead and are never used; the row at pos is taken
  // from LDS), so all of them are in flight together.
  auto load_pass = [&](int ps, uint4 (&kr)[4], uint4 (&vr)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int jj = ps * kPass + 16 * i + 4 * w + gq;
      const size_t row = (size_t)(jj < n ? t0 + jj : t0) * SK_HD + 8 * sl;
      kr[i] = gload4((const uint4*)(Kh + row));
      vr[i] = gload4((const uint4*)(Vh + row));
    }
  };
  // this step's inputs first (the wait for them must not also wait for the cache rows), then every cache row
  const float c = a.rope[(size_t)pos * SK_HD + (d & 63)], s = a.rope[(size_t)pos * SK_HD + 64 + (d & 63)];
  const float qv = qrow[(2 * kvh + p) * SK_HD + d];
  const float kv = has_pos ? qrow[a.nq * SK_HD + p * a.nkv * SK_HD + kvh * SK_HD + d] : 0.f;
  const float qw = a.qn[d], kw = a.kn[d];
  uint4 kr[kAttnPasses][4], vr[kAttnPasses][4];
#pragma unroll
  for (int ps = 0; ps < kAttnPasses; ps++) load_pass(ps, kr[ps], vr[ps]);
  // q of both heads (and, in the split holding pos, this step's k / v): per-head RMSNorm, RoPE, bf16 append
  {
    const float sq = wave_sum(qv * qv), sk = wave_sum(kv * kv);
    if (lane == 0) { red[w] = sq; red[4 + w] = sk; }
    __syncthreads();
    qsh[p][d] = qv * rsqrtf((red[2 * p] + red[2 * p + 1]) / SK_HD + a.eps) * qw;
    if (has_pos) {
      if (p == 0) ksh[d] = kv * rsqrtf((red[4] + red[5]) / SK_HD + a.eps) * kw;
      else vsh[d] = bf2f(f2bf(kv));
    }
    __syncthreads();
    const float qr = (qsh[p][d] * c + (d < 64 ? -qsh[p][d + 64] : qsh[p][d - 64]) * s) * kInvSqrtHd;
    float krot = 0.f;
    if (has_pos && p == 0) krot = bf2f(f2bf(ksh[d] * c + (d < 64 ? -ksh[d + 64] : ksh[d - 64]) * s));
    __syncthreads();
    qsh[p][d] = qr;
    if (has_pos) {
      if (p == 0) { ksh[d] = krot; Kh[(size_t)pos * SK_HD + d] = f2bf(krot); }
      else Vh[(size_t)pos * SK_HD + d] = f2bf(vsh[d]);
    }
    __syncthreads();
  }
  float q0[8], q1[8];
#pragma unroll
  for (int e = 0; e < 8; e++) { q0[e] = qsh[0][8 * sl + e]; q1[e] = qsh[1][8 * sl + e]; }
  float m = -INFINITY, l = 0.f, o = 0.f;  // running partial of head p, dim d
#pragma unroll
  for (int ps = 0; ps < kAttnPasses; ps++) {
    if (ps >= npass) break;  // uniform over the block
    const int base = ps * kPass, np = min(kPass, n - base);
    // scores of both heads
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int jl = 16 * i + 4 * w + gq;
      float k8[8];
      if (base + jl < n && t0 + base + jl == pos) {
#pragma unroll
        for (int e = 0; e < 8; e++) k8[e] = ksh[8 * sl + e];
      } else {
        unpack8(kr[ps][i], k8);
      }
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) { s0 = __builtin_fmaf(q0[e], k8[e], s0); s1 = __builtin_fmaf(q1[e], k8[e], s1); }
      s0 = row16_sum(s0);
      s1 = row16_sum(s1);
      if (sl == 0 && jl < np) { sc[0][jl] = s0; sc[1][jl] = s1; }
    }
    __syncthreads();
    // pass softmax statistics per head (threads 0-127: head 0, 128-255: head 1)
    const float sv = d < np ? sc[p][d] : -INFINITY;
    const float mx = wave_max(sv);
    if (lane == 0) red[8 + w] = mx;
    __syncthreads();
    const float mp = fmaxf(red[8 + 2 * p], red[8 + 2 * p + 1]);
    const float ev = d < np ? expf(sv - mp) : 0.f;
    const float se = wave_sum(ev);
    if (d < np) sc[p][d] = ev;
    if (lane == 0) red[12 + w] = se;
    __syncthreads();
    const float lp = red[12 + 2 * p] + red[12 + 2 * p + 1];
    // Σ p_j v_j for both heads
    float a0[8], a1[8];
#pragma unroll
    for (int e = 0; e < 8; e++) { a0[e] = 0.f; a1[e] = 0.f; }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int jl = 16 * i + 4 * w + gq;
      if (jl < np) {
        float v8[8];
        if (t0 + base + jl == pos) {
#pragma unroll
          for (int e = 0; e < 8; e++) v8[e] = vsh[8 * sl + e];
        } else {
          unpack8(vr[ps][i], v8);
        }
        const float e0 = sc[0][jl], e1 = sc[1][jl];
#pragma unroll
        for (int e = 0; e < 8; e++) { a0[e] = __builtin_fmaf(e0, v8[e], a0[e]); a1[e] = __builtin_fmaf(e1, v8[e], a1[e]); }
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e++) { opart[w][gq][sl][e] = a0[e]; opart[w][gq][sl][8 + e] = a1[e]; }
    __syncthreads();
    float op = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ww++)
#pragma unroll
      for (int gg = 0; gg < 4; gg++) op += opart[ww][gg][d >> 3][p * 8 + (d & 7)];
    // fold the pass into the running partial
    const float mn = fmaxf(m, mp);
    const float fo = m == -INFINITY ? 0.f : expf(m - mn), fp = expf(mp - mn);
    o = o * fo + op * fp;
    l = l * fo + lp * fp;
    m = mn;
    __syncthreads();  // sc / opart are rewritten by the next pass
  }

  if (ns == 1) {  // the whole cache in this block: the output directly, nothing to merge
    store_terms(a.att, ap, (size_t)b * a.nq * SK_HD + (2 * kvh + p) * SK_HD + d, l > 0.f ? o / l : 0.f);
    return;
  }
  // publish the partial for k_bmerge
  float* pp = a.part + ((bg * 2 + p) * kAttnSplitMax + split) * kPart;  // plain stores: k_bmerge is another launch
  if (d == 0) { pp[0] = m; pp[1] = l; }
  pp[2 + d] = o;
}

// Block (stream b, kv head g): the log-sum-exp merge of k_battn's partials of (b, g) in split order (thread (p, d): q
// head 2 g + p, dim d), written as bf16 term planes. Streams past their cache and streams of one split were handled
// by k_battn.
__global__ __launch_bounds__(kThreads) void k_bmerge(AttnArgs a) {
  __shared__ float mls[2][kAttnSplitMax][2];
  const int bg = blockIdx.x, b = bg / a.nkv, kvh = bg % a.nkv;
  const int t = threadIdx.x, p = t >> 7, d = t & (SK_HD - 1);
  const int64_t pos64 = a.pos[b];
  if (pos64 < 0 || pos64 >= a.max_len) return;
  const int ns = ((int)pos64 + kAttnChunk) / kAttnChunk;
  if (ns == 1) return;
  if (t < 2 * ns) {
    const int pp = t / ns, cc = t % ns;
    const float* q = a.part + ((bg * 2 + pp) * kAttnSplitMax + cc) * kPart;
    mls[pp][cc][0] = q[0];
    mls[pp][cc][1] = q[1];
  }
  float oc[kAttnSplitMax];
  const float* po = a.part + (bg * 2 + p) * kAttnSplitMax * kPart + 2 + d;
#pragma unroll
  for (int k = 0; k < kAttnSplitMax; k++) oc[k] = po[(k < ns ? k : 0) * kPart];
  __syncthreads();
  float M = -INFINITY;
  for (int cc = 0; cc < ns; cc++) M = fmaxf(M, mls[p][cc][0]);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int k = 0; k < kAttnSplitMax; k++) {
    if (k < ns && mls[p][k][0] != -INFINITY) {
      const float f = expf(mls[p][k][0] - M);
      L = __builtin_fmaf(f, mls[p][k][1], L);
      O = __builtin_fmaf(f, oc[k], O);
    }
  }
  const size_t ap = (size_t)kM * a.nq * SK_HD;
  store_terms(a.att, ap, (size_t)b * a.nq * SK_HD + (2 * kvh + p) * SK_HD + d, L > 0.f ? O / L : 0.f);
}

// ---- greedy pick + embedding of the next input ---------------------------------------------------------------
// Block b: argmax of logits row b (largest value, lowest index on ties, NaN never wins; qwen3/sampler.py:114-149)
// when pick != 0, else the stored id; then h[b] = emb[id] (bf16 -> fp32), the input planes of bf16(h ⊙ nw0) and
// the row's sum of squares (one partial) for the first layer's RMSNorm.
struct PickArgs {
  const float* logits;  // [16][V]
  int V, H, pick, max_frames;
  int64_t* ids;         // [batch]
  int64_t* pos;         // [batch]
  int64_t* codes;       // [max_frames][16]
  int64_t* nstep;       // [batch]
  const bf16_t* emb;    // [V][H]
  const float* nw0;     // [H]
  float* h;             // [16][H]
  bf16_t* xa;           // planes [kTerms][16][H]
  float* ssa;           // [1][16]
  int* err;
};

__global__ __launch_bounds__(kThreads) void k_bpick(PickArgs a) {
  __shared__ float bv[kThreads];
  __shared__ int bi[kThreads];
  __shared__ float red[kThreads / SK_WAVE];
  __shared__ int id_s;
  const int b = blockIdx.x, t = threadIdx.x;
  if (a.pick) {
    const float* lg = a.logits + (size_t)b * a.V;
    float best = 0.f;
    int bidx = -1;
    for (int k = t; k < a.V; k += kThreads) {
      const float v = lg[k];
      if (v == v && (bidx < 0 || v > best)) { best = v; bidx = k; }
    }
    bv[t] = best;
    bi[t] = bidx;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
      if (t < s) {
        const int j2 = bi[t + s];
        if (j2 >= 0 && (bi[t] < 0 || bv[t + s] > bv[t] || (bv[t + s] == bv[t] && j2 < bi[t]))) {
          bv[t] = bv[t + s];
          bi[t] = j2;
        }
      }
      __syncthreads();
    }
    if (t == 0) {
      const int id = bi[0] < 0 ? 0 : bi[0];
      id_s = id;
      a.ids[b] = id;
      const int64_t f = a.nstep[b];
      if (f >= 0 && f < a.max_frames) a.codes[f * kM + b] = id;
      else atomicCAS(a.err, 0, 6);
      a.nstep[b] = f + 1;
      a.pos[b] = a.pos[b] + 1;
    }
  } else if (t == 0) {
    int64_t id = a.ids[b];
    if (id < 0 || id >= a.V) { atomicCAS(a.err, 0, 5); id = 0; }
    id_s = (int)id;
  }
  __syncthreads();
  const int id = id_s;
  const bf16_t* row = a.emb + (size_t)id * a.H;
  float ss = 0.f;
  for (int k = t; k < a.H; k += kThreads) {
    const float v = bf2f(row[k]);
    a.h[(size_t)b * a.H + k] = v;
    store_terms(a.xa, (size_t)kM * a.H, (size_t)b * a.H + k, v * a.nw0[k]);
    ss = __builtin_fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) red[t >> 6] = ss;
  __syncthreads();
  if (t == 0) a.ssa[b] = (red[0] + red[1]) + (red[2] + red[3]);
}

// ---- dispatch ------------------------------------------------------------------------------------------------
// Launch plan: R row groups per wave (2 from N = 8192 rows up, else 1), slices of CW 64-wide chunks (8, halved while
// the grid has fewer than kMinWg workgroups), S = K / (64 CW) slices, NB row blocks of 4 R groups. Measured on the
// 1.7B step (16 streams): slices of 16 chunks (96 KB of LDS, fewer slices) 7657 and a minimum of 96 workgroups 7958
// against 7992 stream-frames/s.
constexpr int kMinWg = 192;
struct Plan { int R, CW, S, NB; };
Plan plan(int N, int K) {
  Plan pl;
  pl.R = N >= 8192 ? 2 : 1;
  pl.NB = (N / 16 + 4 * pl.R - 1) / (4 * pl.R);
  pl.CW = 8;
  while (pl.CW > 2 && (K % (64 * pl.CW) != 0 ||
                       (pl.NB * (K / (64 * pl.CW)) < kMinWg && K / (32 * pl.CW) <= kMaxSlices)))
    pl.CW /= 2;
  pl.S = K / (64 * pl.CW);
  return pl;
}
int64_t part_floats(int N, int K) {
  const Plan pl = plan(N, K);
  return pl.S > 1 ? (int64_t)pl.S * (N / 16) * 256 : 0;
}
template <int OUT, int R>
hipError_t launch_cw(const GemmArgs& p, const Plan& pl, hipStream_t st) {
  const dim3 grid(pl.NB, pl.S);
  switch (pl.CW) {
    case 2: hipLaunchKernelGGL((k_bgemm<OUT, R, 2>), grid, dim3(kThreads), 0, st, p); break;
    case 4: hipLaunchKernelGGL((k_bgemm<OUT, R, 4>), grid, dim3(kThreads), 0, st, p); break;
    case 8: hipLaunchKernelGGL((k_bgemm<OUT, R, 8>), grid, dim3(kThreads), 0, st, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}
bool k_supported(int K) { return K == 512 || K == 1024 || K == 2048 || K == 3072 || K == 4096 || K == 6144; }

hipError_t launch_gemm(GemmArgs p, int mode, hipStream_t st) {
  const Plan pl = plan(p.N, p.K);
  p.S = pl.S;
  if (mode == kOutF32) return pl.R == 2 ? launch_cw<kOutF32, 2>(p, pl, st) : launch_cw<kOutF32, 1>(p, pl, st);
  if (mode == kOutSwiglu) return pl.R == 2 ? launch_cw<kOutSwiglu, 2>(p, pl, st) : launch_cw<kOutSwiglu, 1>(p, pl, st);
  return pl.R == 2 ? launch_cw<kOutAcc, 2>(p, pl, st) : launch_cw<kOutAcc, 1>(p, pl, st);
}

int check_gemm(const GemmArgs& p, int mode) {
  if (!p.x || !p.w || !p.s || (!p.out && mode != kOutSwiglu)) return SK_EINVAL;
  if (p.N <= 0 || p.N % 16 || !k_supported(p.K)) return SK_EINVAL;
  if (p.ssp && p.np < 1) return SK_EINVAL;
  if (mode == kOutSwiglu && (!p.act || p.N % 32)) return SK_EINVAL;
  if (mode == kOutAcc && (!p.xn || !p.nw || !p.ssp_out)) return SK_EINVAL;
  if (mode < 0 || mode > kOutAcc) return SK_EINVAL;
  if (!SK_ALIGNED16(p.x) || !SK_ALIGNED16(p.w)) return SK_EINVAL;
  return SK_OK;
}

// workspace layout
struct Ws {
  int64_t err, h, xa, xb, ssa, ssb, qkv, att, act, logits, part, gpart, gctr, total;
};
int64_t up256(int64_t v) { return (v + 255) / 256 * 256; }
Ws ws_layout(int H, int I, int nq, int nkv, int V) {
  Ws w;
  int64_t o = 0;
  auto take = [&](int64_t bytes) { const int64_t at = o; o += up256(bytes); return at; };
  w.err = take(256);
  w.h = take((int64_t)kM * H * 4);
  w.xa = take((int64_t)kTerms * kM * H * 2);
  w.xb = take((int64_t)kTerms * kM * H * 2);
  w.ssa = take((int64_t)(H / 16) * kM * 4);
  w.ssb = take((int64_t)(H / 16) * kM * 4);
  w.qkv = take((int64_t)kM * (nq + 2 * nkv) * SK_HD * 4);
  w.att = take((int64_t)kTerms * kM * nq * SK_HD * 2);
  w.act = take((int64_t)kTerms * kM * I * 2);
  w.logits = take((int64_t)kM * V * 4);
  w.part = take((int64_t)kM * nkv * 2 * kAttnSplitMax * kPart * 4);
  const int nqkv = (nq + 2 * nkv) * SK_HD;
  int64_t pf = 0, nmax = 0;
  const int shapes[5][2] = {{nqkv, H}, {H, nq * SK_HD}, {2 * I, H}, {H, I}, {V, H}};
  for (const auto& sh : shapes) {
    pf = pf > part_floats(sh[0], sh[1]) ? pf : part_floats(sh[0], sh[1]);
    nmax = nmax > sh[0] ? nmax : sh[0];
  }
  w.gpart = take(pf * 4);
  w.gctr = take(nmax / 16 * 4);
  w.total = o;
  return w;
}

}  // namespace

extern "C" int sk_tile_weights(const void* w, void* tiled, int N, int K, void* stream) {
  if (!w || !tiled || N <= 0 || K <= 0 || N % 16 || K % 64) return sk_set_error(SK_EINVAL, "sk_tile_weights: bad arguments");
  if (!SK_ALIGNED16(w) || !SK_ALIGNED16(tiled)) return sk_set_error(SK_EINVAL, "sk_tile_weights: pointers must be 16-byte aligned");
  const size_t slots = (size_t)N * K / 16;
  hipLaunchKernelGGL(k_tile, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (const int8_t*)w, (int8_t*)tiled, N, K);
  return sk_check_launch(hipGetLastError(), "sk_tile_weights");
}

extern "C" int64_t sk_bgemm_workspace_size(int N, int K) {
  if (N <= 0 || N % 16 || !k_supported(K)) return 0;
  return up256(part_floats(N, K) * 4) + up256((int64_t)N / 16 * 4);
}

extern "C" int sk_bgemm(const void* x, const float* ssp, int np, float eps, const void* w_tiled, const uint16_t* s, int N,
                        int K, int mode, float* out, void* act, void* xn, const float* nw, float* ssp_out,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  GemmArgs p{(const bf16_t*)x, ssp, np, eps, (const uint8_t*)w_tiled, s, N, K, out, (bf16_t*)act, (bf16_t*)xn, nw, ssp_out,
             1, nullptr, nullptr};
  if (check_gemm(p, mode)) return sk_set_error(SK_EINVAL, "sk_bgemm: bad shape, mode or pointer");
  if (!workspace || !SK_ALIGNED16(workspace)) return sk_set_error(SK_EINVAL, "sk_bgemm: workspace must be 16-byte aligned");
  if (workspace_bytes < sk_bgemm_workspace_size(N, K)) return sk_set_error(SK_EWORKSPACE, "sk_bgemm: workspace too small");
  p.part = (float*)workspace;
  p.counters = (unsigned*)((char*)workspace + up256(part_floats(N, K) * 4));
  return sk_check_launch(launch_gemm(p, mode, (hipStream_t)stream), "sk_bgemm");
}

extern "C" int sk_batch_terms(void) { return kTerms; }

extern "C" int64_t sk_batch_workspace_size(int hidden, int inter, int nq, int nkv, int vocab) {
  if (hidden <= 0 || inter <= 0 || nq <= 0 || nkv <= 0 || vocab <= 0) return 0;
  return ws_layout(hidden, inter, nq, nkv, vocab).total;
}

namespace {
int check_batch(const sk_batch_desc* d) {
  if (!d) return sk_set_error(SK_EINVAL, "sk_batch: null descriptor");
  const int H = d->hidden, I = d->inter;
  if (d->batch < 1 || d->batch > kM) return sk_set_error(SK_EINVAL, "sk_batch: batch must be 1..16");
  if (d->nkv <= 0 || d->nq != 2 * d->nkv) return sk_set_error(SK_EINVAL, "sk_batch: needs nq == 2 nkv (head_dim 128)");
  if (!k_supported(H) || !k_supported(I) || !k_supported(d->nq * SK_HD) || H % 16)
    return sk_set_error(SK_EINVAL, "sk_batch: hidden / inter / nq*128 must be 512, 1024, 2048, 3072, 4096 or 6144");
  if (d->vocab <= 0 || d->vocab % 16) return sk_set_error(SK_EINVAL, "sk_batch: vocab must be a positive multiple of 16");
  if (d->max_len <= 0 || d->max_len > kAttnChunk * kAttnSplitMax) return sk_set_error(SK_EINVAL, "sk_batch: max_len must be 1..4096");
  if (d->n_layers <= 0 || !d->layers || !d->norm || !d->head_w || !d->head_s || !d->emb || !d->rope || !d->ids || !d->pos ||
      !d->codes || !d->nstep || d->max_frames <= 0 || !d->workspace)
    return sk_set_error(SK_EINVAL, "sk_batch: null pointer or bad count");
  if (!SK_ALIGNED16(d->workspace)) return sk_set_error(SK_EINVAL, "sk_batch: workspace must be 16-byte aligned");
  if (d->workspace_bytes < sk_batch_workspace_size(H, I, d->nq, d->nkv, d->vocab))
    return sk_set_error(SK_EWORKSPACE, "sk_batch: workspace too small");
  for (int l = 0; l < d->n_layers; l++) {
    const sk_layer_desc& L = d->layers[l];
    if (!L.qkv_w || !L.qkv_s || !L.o_w || !L.o_s || !L.gu_w || !L.gu_s || !L.down_w || !L.down_s || !L.in_norm ||
        !L.post_norm || !L.qn || !L.kn || !L.kc || !L.vc)
      return sk_set_error(SK_EINVAL, "sk_batch: null pointer in a layer descriptor");
    if (!SK_ALIGNED16(L.kc) || !SK_ALIGNED16(L.vc)) return sk_set_error(SK_EINVAL, "sk_batch: caches must be 16-byte aligned");
  }
  return SK_OK;
}

hipError_t embed_launch(const sk_batch_desc* d, int pick, hipStream_t st) {
  char* ws = (char*)d->workspace;
  const Ws w = ws_layout(d->hidden, d->inter, d->nq, d->nkv, d->vocab);
  PickArgs a{(const float*)(ws + w.logits), d->vocab, d->hidden, pick, d->max_frames, d->ids, d->pos, d->codes, d->nstep,
             (const bf16_t*)d->emb, d->layers[0].in_norm, (float*)(ws + w.h), (bf16_t*)(ws + w.xa), (float*)(ws + w.ssa),
             (int*)(ws + w.err)};
  hipLaunchKernelGGL(k_bpick, dim3(d->batch), dim3(kThreads), 0, st, a);
  return hipGetLastError();
}
}  // namespace

extern "C" int64_t sk_batch_attn_workspace_size(int nkv) {
  if (nkv <= 0) return 0;
  return up256(256) + up256((int64_t)kM * nkv * 2 * kAttnSplitMax * kPart * 4);
}

extern "C" int sk_batch_attn(const float* qkv, const float* qn, const float* kn, float eps, const float* rope, void* Kc,
                             void* Vc, const int64_t* pos, int batch, int max_len, int nq, int nkv, void* att,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  if (!qkv || !qn || !kn || !rope || !Kc || !Vc || !pos || !att || !workspace)
    return sk_set_error(SK_EINVAL, "sk_batch_attn: null pointer");
  if (batch < 1 || batch > kM || nkv <= 0 || nq != 2 * nkv || max_len <= 0 || max_len > kAttnChunk * kAttnSplitMax)
    return sk_set_error(SK_EINVAL, "sk_batch_attn: needs batch 1..16, nq == 2 nkv, max_len 1..4096");
  if (!SK_ALIGNED16(Kc) || !SK_ALIGNED16(Vc) || !SK_ALIGNED16(workspace))
    return sk_set_error(SK_EINVAL, "sk_batch_attn: caches and workspace must be 16-byte aligned");
  if (workspace_bytes < sk_batch_attn_workspace_size(nkv)) return sk_set_error(SK_EWORKSPACE, "sk_batch_attn: workspace too small");
  char* ws = (char*)workspace;
  const int64_t part = up256(256);
  AttnArgs at{qkv, qn, kn, eps, rope, (bf16_t*)Kc, (bf16_t*)Vc, pos, max_len, nq, nkv, (bf16_t*)att,
              (float*)(ws + part), (int*)ws};
  hipLaunchKernelGGL(k_battn, dim3(batch * nkv, (max_len + kAttnChunk - 1) / kAttnChunk), dim3(kThreads), 0,
                     (hipStream_t)stream, at);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_bmerge, dim3(batch * nkv), dim3(kThreads), 0, (hipStream_t)stream, at);
    e = hipGetLastError();
  }
  return sk_check_launch(e, "sk_batch_attn");
}

extern "C" int sk_batch_embed(const sk_batch_desc* d, void* stream) {
  int rc = check_batch(d);
  if (rc) return rc;
  return sk_check_launch(embed_launch(d, 0, (hipStream_t)stream), "sk_batch_embed");
}

extern "C" int sk_batch_frame(const sk_batch_desc* d, void* stream) {
  int rc = check_batch(d);
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  char* ws = (char*)d->workspace;
  const int H = d->hidden, I = d->inter, nq = d->nq, nkv = d->nkv, V = d->vocab;
  const Ws w = ws_layout(H, I, nq, nkv, V);
  float* h = (float*)(ws + w.h);
  bf16_t* xa = (bf16_t*)(ws + w.xa);
  bf16_t* xb = (bf16_t*)(ws + w.xb);
  float* ssa = (float*)(ws + w.ssa);
  float* ssb = (float*)(ws + w.ssb);
  float* qkv = (float*)(ws + w.qkv);
  bf16_t* att = (bf16_t*)(ws + w.att);
  bf16_t* act = (bf16_t*)(ws + w.act);
  float* logits = (float*)(ws + w.logits);
  float* gpart = (float*)(ws + w.gpart);
  unsigned* gctr = (unsigned*)(ws + w.gctr);
  const int nqkv = (nq + 2 * nkv) * SK_HD;
  hipError_t e = hipSuccess;
  for (int l = 0; l < d->n_layers && e == hipSuccess; l++) {
    const sk_layer_desc& L = d->layers[l];
    const int np_a = l == 0 ? 1 : H / 16;
    GemmArgs g1{xa, ssa, np_a, d->eps, (const uint8_t*)L.qkv_w, L.qkv_s, nqkv, H, qkv, nullptr, nullptr, nullptr, nullptr,
                1, gpart, gctr};
    e = launch_gemm(g1, kOutF32, st);
    if (e != hipSuccess) break;
    AttnArgs at{qkv, L.qn, L.kn, d->eps, d->rope, (bf16_t*)L.kc, (bf16_t*)L.vc, d->pos, d->max_len, nq, nkv, att,
                (float*)(ws + w.part), (int*)(ws + w.err)};
    hipLaunchKernelGGL(k_battn, dim3(d->batch * nkv, (d->max_len + kAttnChunk - 1) / kAttnChunk), dim3(kThreads), 0, st, at);
    e = hipGetLastError();
    if (e != hipSuccess) break;
    hipLaunchKernelGGL(k_bmerge, dim3(d->batch * nkv), dim3(kThreads), 0, st, at);
    e = hipGetLastError();
    if (e != hipSuccess) break;
    GemmArgs g2{att, nullptr, 0, d->eps, (const uint8_t*)L.o_w, L.o_s, H, nq * SK_HD, h, nullptr, xb, L.post_norm, ssb,
                1, gpart, gctr};
    e = launch_gemm(g2, kOutAcc, st);
    if (e != hipSuccess) break;
    GemmArgs g3{xb, ssb, H / 16, d->eps, (const uint8_t*)L.gu_w, L.gu_s, 2 * I, H, nullptr, act, nullptr, nullptr, nullptr,
                1, gpart, gctr};
    e = launch_gemm(g3, kOutSwiglu, st);
    if (e != hipSuccess) break;
    const float* nw_next = l + 1 < d->n_layers ? d->layers[l + 1].in_norm : d->norm;
    GemmArgs g4{act, nullptr, 0, d->eps, (const uint8_t*)L.down_w, L.down_s, H, I, h, nullptr, xa, nw_next, ssa,
                1, gpart, gctr};
    e = launch_gemm(g4, kOutAcc, st);
    if (e != hipSuccess) break;
    if (d->layer_out)
      e = hipMemcpyAsync(d->layer_out + (size_t)l * kM * H, h, (size_t)kM * H * 4, hipMemcpyDeviceToDevice, st);
  }
  if (e == hipSuccess) {
    GemmArgs gh{xa, ssa, H / 16, d->eps, (const uint8_t*)d->head_w, d->head_s, V, H, logits, nullptr, nullptr, nullptr,
                nullptr, 1, gpart, gctr};
    e = launch_gemm(gh, kOutF32, st);
  }
  if (e == hipSuccess && d->logits) e = hipMemcpyAsync(d->logits, logits, (size_t)kM * V * 4, hipMemcpyDeviceToDevice, st);
  if (e == hipSuccess) e = embed_launch(d, 1, st);
  return sk_check_launch(e, "sk_batch_frame");
}
