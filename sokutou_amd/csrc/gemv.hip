// M=1 weight-only GEMV for the talker projections (qkv, o, gate/up, down, codec head).
//
// Replaces the reference's `rms_gemv` / `gemv` kernels (qwen3/kernels.py:143-310). One 256-thread block is four
// wave64s; each wave owns RPW consecutive rows. Lane l reads 16-byte chunks l, l+64, ... of every row it owns, so
// a wave's loads of one row are one contiguous 1 KiB stretch of HBM (global_load_dwordx4, nontemporal for
// weights that are read once per frame). The first chunks are requested before the input vector is staged in
// LDS, so the weight stream starts at the top of the kernel. Dequantisation happens in registers
// (v_cvt_f32_i32 with a sign-extended byte select per weight, then v_fmac), and each row's partial sums are
// reduced across the wave with DPP row operations.
#include "common.h"
#include "internal.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * SK_WAVE;
constexpr int kU = 4;  // chunks per lane kept in flight per row

template <int POL>
__device__ __forceinline__ uint4 ldw(const uint4* p) {
  if constexpr (POL == 1) return ld_stream(p);
  else return *p;
}

// mode: 0 write, 1 accumulate into out, 2 SwiGLU over interleaved gate/up rows (out[row/2]).
template <int WD, int RPW, int POL>
__global__ __launch_bounds__(kThreads) void k_gemv(const float* __restrict__ x, const float* __restrict__ nw, float eps,
                                                   const uint8_t* __restrict__ W, const uint16_t* __restrict__ S,
                                                   const float* __restrict__ bias, float* __restrict__ out, int N, int K,
                                                   int mode) {
  extern __shared__ float xs[];
  constexpr int E = WdInfo<WD>::E;
  const int w = threadIdx.x / SK_WAVE, lane = threadIdx.x % SK_WAVE;
  const int row0 = (blockIdx.x * kWaves + w) * RPW;
  const int nc = K / E;  // 16-byte chunks per row
  const size_t row_bytes = (size_t)K * WdInfo<WD>::BYTES;
  const uint4* wr[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int row = row0 + r < N ? row0 + r : 0;
    wr[r] = (const uint4*)(W + (size_t)row * row_bytes);
  }
  uint4 v[kU][RPW];
#pragma unroll
  for (int u = 0; u < kU; u++) {
    const int c = lane + u * SK_WAVE;
#pragma unroll
    for (int r = 0; r < RPW; r++)
      if (c < nc) v[u][r] = ldw<POL>(wr[r] + c);
  }
  // stage the input (times the norm weight) and, for the fused RMSNorm, the per-wave sum of squares of x
  float inv = 1.f;
  if (nw) {
    float ss = 0.f;
    for (int i = lane * 4; i < K; i += SK_WAVE * 4) {
      float4 a = *(const float4*)(x + i);
      ss += a.x * a.x + a.y * a.y + a.z * a.z + a.w * a.w;
    }
    inv = rsqrtf(wave_sum(ss) / K + eps);
    for (int i = threadIdx.x * 4; i < K; i += kThreads * 4) {
      float4 a = *(const float4*)(x + i), b = *(const float4*)(nw + i);
      *(float4*)(xs + i) = make_float4(a.x * b.x, a.y * b.y, a.z * b.z, a.w * b.w);
    }
  } else {
    for (int i = threadIdx.x * 4; i < K; i += kThreads * 4) *(float4*)(xs + i) = *(const float4*)(x + i);
  }
  __syncthreads();
  int rs[RPW];  // row index for scale reads, clamped like the weight pointers
#pragma unroll
  for (int r = 0; r < RPW; r++) rs[r] = row0 + r < N ? row0 + r : 0;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) acc[r] = 0.f;
  for (int base = 0; base < nc; base += kU * SK_WAVE) {
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int c = base + lane + u * SK_WAVE;
      if (c < nc) {
#pragma unroll
        for (int r = 0; r < RPW; r++) acc[r] += chunk_dot<WD>(v[u][r], xs + c * E, S, rs[r], K, c);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int c = base + (kU + u) * SK_WAVE + lane;
#pragma unroll
      for (int r = 0; r < RPW; r++)
        if (c < nc) v[u][r] = ldw<POL>(wr[r] + c);
    }
  }
  float y[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) y[r] = wave_sum(acc[r]) * row_scale<WD>(S, rs[r]) * inv;
  if (lane != 0) return;
  if (mode == 2) {
#pragma unroll
    for (int r = 0; r + 1 < RPW; r += 2)
      if (row0 + r + 1 < N) out[(row0 + r) >> 1] = silu_mul(y[r], y[r + 1]);
    return;
  }
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const int row = row0 + r;
    if (row >= N) break;
    float o = y[r];
    if (bias) o += bias[row];
    if (mode == 1) o += out[row];
    out[row] = o;
  }
}

template <int WD, int RPW, int POL>
hipError_t launch_rpw(const float* x, const float* nw, float eps, const void* W, const uint16_t* S, const float* bias,
                      float* out, int N, int K, int mode, hipStream_t st) {
  const int rows_per_block = kWaves * RPW;
  dim3 grid((N + rows_per_block - 1) / rows_per_block);
  hipLaunchKernelGGL((k_gemv<WD, RPW, POL>), grid, dim3(kThreads), K * sizeof(float), st, x, nw, eps,
                     (const uint8_t*)W, S, bias, out, N, K, mode);
  return hipGetLastError();
}

template <int WD, int POL>
hipError_t launch_wd(const float* x, const float* nw, float eps, const void* W, const uint16_t* S, const float* bias,
                     float* out, int N, int K, int mode, hipStream_t st) {
  // Pick the rows per wave so that the grid has at least 256 blocks (one per CU) when N allows; SwiGLU needs an
  // even count so gate and up rows meet in one wave.
  if (N >= 256 * kWaves * 4) return launch_rpw<WD, 4, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
  if (N >= 256 * kWaves * 2 || mode == 2) return launch_rpw<WD, 2, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
  return launch_rpw<WD, 1, POL>(x, nw, eps, W, S, bias, out, N, K, mode, st);
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
