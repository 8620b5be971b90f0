// M=1 weight-only GEMV for the talker projections (qkv, o, gate/up, down, codec head): sk_rms_gemv and sk_gemv,
// replacing the reference's `rms_gemv` / `gemv` (qwen3/kernels.py:255-310; math of gemv_core 143-253).
//
// Design for CDNA4 (wave64, 256 CUs):
//  * One workgroup is ONE wave and owns 4 * RG consecutive rows. The wave is four 16-lane groups; group g takes rows
//    r0 + g + 4 k (k < RG) and its 16 lanes split K: lane q reads 16-byte chunks q, q + 16, q + 32, ... of each of its
//    rows. A row's result is a 16-lane DPP row sum (four DPP steps; no cross-row or cross-wave reduction). Small
//    projections (1024 rows) still launch 256 workgroups and fill the chip.
//  * Each wave stages the input itself in LDS, chunk-major: quarter j (4 floats) of chunk c sits at 16-byte slot
//    j * nc + c. In one read instruction the 16 lanes of a group read 16 consecutive slots and the four groups read
//    the same slots (broadcast), and the staging writes are consecutive slots too: no bank conflicts either way, and
//    no workgroup barrier (one wave). The fused RMSNorm's sum of squares comes from the same staging reads.
//  * Weights are loaded P (kP) chunks per lane and row at a time, double-buffered across passes (two register sets used
//    alternately, never copied, so no pass waits for younger loads). The first pass is requested before the input is
//    staged. Loads past the end of a row are clamped to its first chunk and their products dropped, so every load
//    is unconditional.
//  * Dequantisation in registers: int8 -> fp32 per byte, fp32 FMA; i8row applies the bf16 row scale after the row
//    sum, i8g32 the fp16 scale of each 32-element group per 16-element chunk; the RMSNorm factor multiplies the
//    result (the reference's order, qwen3/kernels.py:180-186, 224).
#include "common.h"
#include "internal.h"

namespace {

constexpr int kGroups = 4;  // 16-lane row groups per wave

template <int POL>
__device__ __forceinline__ uint4 ldw(const uint4* p) {
  if constexpr (POL == 1) return ld_stream(p);
  else return *p;
}

// Dot of one 16-byte weight chunk with its E inputs, held as E / 4 float4 quarters.
template <int WD>
__device__ __forceinline__ float chunk_dot4(uint4 v, const float4* xv) {
  if constexpr (WD == SK_WD_I8ROW || WD == SK_WD_I8G32) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      a = __builtin_fmaf((float)(int8_t)(w[j]), xv[j].x, a);
      a = __builtin_fmaf((float)(int8_t)(w[j] >> 8), xv[j].y, a);
      a = __builtin_fmaf((float)(int8_t)(w[j] >> 16), xv[j].z, a);
      a = __builtin_fmaf((float)(int8_t)(w[j] >> 24), xv[j].w, a);
    }
    return a;
  } else if constexpr (WD == SK_WD_BF16) {
    float a = bf2f(v.x & 0xffffu) * xv[0].x;
    a = __builtin_fmaf(bf2f(v.x >> 16), xv[0].y, a);
    a = __builtin_fmaf(bf2f(v.y & 0xffffu), xv[0].z, a);
    a = __builtin_fmaf(bf2f(v.y >> 16), xv[0].w, a);
    a = __builtin_fmaf(bf2f(v.z & 0xffffu), xv[1].x, a);
    a = __builtin_fmaf(bf2f(v.z >> 16), xv[1].y, a);
    a = __builtin_fmaf(bf2f(v.w & 0xffffu), xv[1].z, a);
    a = __builtin_fmaf(bf2f(v.w >> 16), xv[1].w, a);
    return a;
  } else {
    float a = __uint_as_float(v.x) * xv[0].x;
    a = __builtin_fmaf(__uint_as_float(v.y), xv[0].y, a);
    a = __builtin_fmaf(__uint_as_float(v.z), xv[0].z, a);
    a = __builtin_fmaf(__uint_as_float(v.w), xv[0].w, a);
    return a;
  }
}

// mode: 0 write, 1 accumulate into out, 2 SwiGLU over interleaved gate/up rows (out[row / 2]).
template <int WD, int RG, int POL, int kP>
__global__ __launch_bounds__(SK_WAVE) void k_gemv(const float* __restrict__ x, const float* __restrict__ nw, float eps,
                                                  const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                                  const float* __restrict__ bias, float* __restrict__ out, int N, int K,
                                                  int mode) {
  constexpr int E = WdInfo<WD>::E, Q = E / 4;  // elements per 16-byte chunk, float4 quarters per chunk
  extern __shared__ float4 xq[];               // staged input: quarter j of chunk c at slot j * nc + c
  const int lane = threadIdx.x, grp = lane >> 4, q = lane & 15;
  const int nc = K / E;  // chunks per row (a multiple of 32: K % 512 == 0)
  const size_t row_bytes = (size_t)K * WdInfo<WD>::BYTES;
  const int r0 = blockIdx.x * kGroups * RG;
  int rows[RG];
  const uint4* wp[RG];
#pragma unroll
  for (int k = 0; k < RG; k++) {
    const int row = r0 + grp + kGroups * k;
    rows[k] = row < N ? row : N - 1;
    wp[k] = (const uint4*)(W + (size_t)rows[k] * row_bytes);
  }
  // pass p covers chunks c = 16 (kP p + i) + q, i < kP; a chunk past the row end is loaded from chunk 0 and dropped
  // (i8g32: the fp16 scale of each chunk's 32-element group comes with it)
  auto load_pass = [&](uint4 (&wv)[RG][kP], uint16_t (&sv)[RG][kP], int p) {
#pragma unroll
    for (int i = 0; i < kP; i++) {
      const int c = 16 * (kP * p + i) + q;
      const int cc = c < nc ? c : 0;
#pragma unroll
      for (int k = 0; k < RG; k++) {
        wv[k][i] = ldw<POL>(wp[k] + cc);
        if constexpr (WD == SK_WD_I8G32) sv[k][i] = S[(size_t)rows[k] * (K >> 5) + (cc >> 1)];
      }
    }
  };
  uint4 wa[RG][kP], wb[RG][kP];
  uint16_t sa[RG][kP], sb[RG][kP];
  load_pass(wa, sa, 0);
  // stage the input (times the norm weight), consecutive slots per instruction; sum of squares for the RMSNorm
  float ss = 0.f;
  const int nslots = nc * Q;
  for (int s = lane; s < nslots; s += SK_WAVE) {
    const int j = s / nc, c = s - j * nc;
    const int e = c * E + 4 * j;  // first element of the quarter
    float4 a = *(const float4*)(x + e);
    if (nw) {
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
      const float4 b = *(const float4*)(nw + e);
      a = make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
    }
    xq[s] = a;
  }
  const float inv = nw ? rsqrtf(wave_sum(ss) / K + eps) : 1.f;
  __syncthreads();  // one wave: orders the LDS writes before the reads
  float acc[RG];
#pragma unroll
  for (int k = 0; k < RG; k++) acc[k] = 0.f;
  auto consume = [&](const uint4 (&wv)[RG][kP], const uint16_t (&sv)[RG][kP], int p) {
#pragma unroll
    for (int i = 0; i < kP; i++) {
      const int c = 16 * (kP * p + i) + q;
      if (c < nc) {
        float4 xv[Q];
#pragma unroll
        for (int j = 0; j < Q; j++) xv[j] = xq[j * nc + c];
#pragma unroll
        for (int k = 0; k < RG; k++) {
          const float d = chunk_dot4<WD>(wv[k][i], xv);
          if constexpr (WD == SK_WD_I8G32) acc[k] = __builtin_fmaf(h2f(sv[k][i]), d, acc[k]);
          else acc[k] += d;
        }
      }
    }
  };
  const int npass = (nc + 16 * kP - 1) / (16 * kP);
  for (int p = 0; p < npass; p += 2) {
    if (p + 1 < npass) load_pass(wb, sb, p + 1);
    consume(wa, sa, p);
    if (p + 1 >= npass) break;
    if (p + 2 < npass) load_pass(wa, sa, p + 2);
    consume(wb, sb, p + 1);
  }
  float y[RG];
#pragma unroll
  for (int k = 0; k < RG; k++) {
    y[k] = row16_sum(acc[k]);
    if constexpr (WD == SK_WD_I8ROW) y[k] *= bf2f(S[rows[k]]);
    y[k] *= inv;
  }
  if (mode == 2) {
    // rows 2n (group 0 / 2) and 2n + 1 (group 1 / 3) meet through a lane permute
#pragma unroll
    for (int k = 0; k < RG; k++) {
      const float up = __shfl_down(y[k], 16);
      const int row = r0 + grp + kGroups * k;
      if (q == 0 && (grp & 1) == 0 && row + 1 < N) out[row >> 1] = silu_mul(y[k], up);
    }
    return;
  }
  if (q != 0) return;
#pragma unroll
  for (int k = 0; k < RG; k++) {
    const int row = r0 + grp + kGroups * k;
    if (row >= N) break;
    float o = y[k];
    if (bias) o += bias[row];
    if (mode == 1) o += out[row];
    out[row] = o;
  }
}

template <int WD, int RG, int POL, int kP>
hipError_t launch_rg(const float* x, const float* nw, float eps, const void* W, const uint16_t* S, const float* bias,
                     float* out, int N, int K, int mode, hipStream_t st) {
  const int rows_per_block = kGroups * RG;
  dim3 grid((N + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((k_gemv<WD, RG, POL, kP>), grid, dim3(SK_WAVE), K * sizeof(float), st, x, nw, eps,
                     (const uint8_t*)W, S, bias, out, N, K, mode);
  return hipGetLastError();
}

template <int WD, int POL>
hipError_t launch_wd(const float* x, const float* nw, float eps, const void* W, const uint16_t* S, const float* bias,
                     float* out, int N, int K, int mode, hipStream_t st) {
  // two rows per group once that still leaves at least 512 workgroups (two waves per CU). With one row per group
  // the few waves per CU keep more of each row in flight, 8 chunks per lane and pass, 16 from K = 3072: the 1.7B
  // talker's bf16 down projection 15.3 -> 11.8 us per call, its o projection 5.4 -> 4.8 (4 chunks before). Two-row
  // groups take 8 chunks only with long rows and few groups (the 1.7B qkv: 6.4 -> 5.5 us per call in bf16); with
  // more groups (gate/up) the deeper pass was slower, 10.6 -> 11.3 us.
  if (N >= 512 * kGroups * 2 && K >= 2048 && N <= 4096)
    return launch_rg<WD, 2, POL, 8>(x, nw, eps, W, S, bias, out, N, K, mode, st);
  if (N >= 512 * kGroups * 2) return launch_rg<WD, 2, POL, 4>(x, nw, eps, W, S, bias, out, N, K, mode, st);
  if (K >= 3072) return launch_rg<WD, 1, POL, 16>(x, nw, eps, W, S, bias, out, N, K, mode, st);
  return launch_rg<WD, 1, POL, 8>(x, nw, eps, W, S, bias, out, N, K, mode, st);
}

template <int POL>
hipError_t launch_pol(const float* x, const float* nw, float eps, const void* W, const uint16_t* S, const float* bias,
                      float* out, int N, int K, int mode, int wd, hipStream_t st) {
  switch (wd) {
    case SK_WD_I8ROW: return launch_wd<SK_WD_I8ROW, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
    case SK_WD_I8G32: return launch_wd<SK_WD_I8G32, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
    case SK_WD_BF16: return launch_wd<SK_WD_BF16, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
    case SK_WD_F32: return launch_wd<SK_WD_F32, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
  }
  return hipErrorInvalidValue;
}

int check_shape(int N, int K, int wd, const void* S) {
  if (N <= 0 || K <= 0) return SK_EINVAL;
  if (K % 512 != 0) return SK_EINVAL;  // same constraint as the reference's _Lin (qwen3/kernels.py:433)
  if (K > SK_MAX_K) return SK_EINVAL;
  if (wd < 0 || wd > SK_WD_F32) return SK_EINVAL;
  if ((wd == SK_WD_I8ROW || wd == SK_WD_I8G32) && !S) return SK_EINVAL;
  return SK_OK;
}

}  // namespace

extern "C" int sk_rms_gemv(const float* h, const float* nw, float eps, const void* W, const uint16_t* S, float* out,
                           int N, int K, int swiglu, int wd, int policy, void* stream) {
  int rc = check_shape(N, K, wd, S);
  if (rc) return sk_set_error(rc, "sk_rms_gemv: bad shape or format");
  if (!h || !nw || !W || !out) return sk_set_error(SK_EINVAL, "sk_rms_gemv: null pointer");
  if (swiglu && (N & 1)) return sk_set_error(SK_EINVAL, "sk_rms_gemv: swiglu needs an even row count");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = policy ? launch_pol<1>(h, nw, eps, W, S, nullptr, out, N, K, swiglu ? 2 : 0, wd, st)
                        : launch_pol<0>(h, nw, eps, W, S, nullptr, out, N, K, swiglu ? 2 : 0, wd, st);
  return sk_check_launch(e, "sk_rms_gemv");
}

extern "C" int sk_gemv(const float* x, const void* W, const uint16_t* S, const float* bias, float* out, int N, int K,
                       int accumulate, int wd, int policy, void* stream) {
  int rc = check_shape(N, K, wd, S);
  if (rc) return sk_set_error(rc, "sk_gemv: bad shape or format");
  if (!x || !W || !out) return sk_set_error(SK_EINVAL, "sk_gemv: null pointer");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = policy ? launch_pol<1>(x, nullptr, 0.f, W, S, bias, out, N, K, accumulate ? 1 : 0, wd, st)
                        : launch_pol<0>(x, nullptr, 0.f, W, S, bias, out, N, K, accumulate ? 1 : 0, wd, st);
  return sk_check_launch(e, "sk_gemv");
}
