// The 1.7B talker's instantiations of the persistent kernel (hidden 2048, intermediate 6144, 8 compute waves) with
// the control wave's polls staged through LDS.
//
// With 8 compute waves every wave of the workgroup gets 168 registers, too few for the control wave to hold a
// polled vector in flight (poll_cells keeps up to 16 loads of 16 bytes per lane outstanding): it spilled them.
// Here the polls of this translation unit read the cells straight from memory into LDS instead (one 1 KB
// global-to-LDS load per 128 cells, none holding a register), check the epochs and copy the values out of LDS.
// The polls are swapped in by explicit specialisations of poll_cells, which apply to this translation unit's
// instantiations only: the 0.6B kernels (frame.hip) keep the register polls and their generated code.
#include "frame_impl.h"

namespace {

// Raw cells of the poll under way, 8 bytes each: the longest polled vector is the intermediate activation.
constexpr int kRawCells = 6144;
__shared__ __attribute__((aligned(16))) uint64_t g_poll_raw[kRawCells];

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

// Waits until cells [idx0, idx0 + n) all carry epoch e, copying the values to dst (swizzled when SW), as
// poll_cells does. Each producer writes its `stride` consecutive cells with one store instruction, so a round
// first probes the last cell of every producer and reads the whole vector only once all of them carry epoch e (a
// failed read of the whole vector costs a round trip and the LDS pass). The read itself checks every cell's epoch:
// the probe only chooses when to read, so `stride` may also be a multiple of the producers' width (a sparser
// probe). Without PROBE every round reads the whole vector. Measured on the 1.7B
// talker: the probe pays for the gate/up activation (48 KB per read) and the local q | k | v exchange, and costs
// 6-9% on the attention output and the o / down outputs (16 KB), which are read whole. n is a multiple of 128 and
// of stride, at most kRawCells; idx0 is even.
template <bool SW, bool PROBE = true>
__device__ __forceinline__ bool poll_cells_lds(const void* cells, uint32_t idx0, int n, int stride, uint32_t e,
                                               float* dst, void* ws, int lane, const Ctx& c, uint32_t code, int f,
                                               int l) {
  const char* base = (const char*)cells + (size_t)idx0 * 8u + (size_t)lane * 16u;
  const int nprod = n / stride;
  for (uint32_t spin = 0;; spin++) {
    bool ready = true;
    if constexpr (PROBE) {
      for (int pr = lane; pr < nprod; pr += 64) {
        const uint32_t cell = idx0 + (uint32_t)((pr + 1) * stride - 1);
        const u32x2 q = __builtin_amdgcn_raw_buffer_load_b64(make_rsrc(cells), cell * 8u, 0, kPolDev);
        ready &= q.y == e;
      }
    }
    if (__all(ready)) {
#pragma unroll 1
      for (int i = 0; i < n / 128; i++)  // not unrolled: unrolled, every load would hold its own address registers
        __builtin_amdgcn_global_load_lds((const void*)(base + (size_t)i * 1024u),
                                         (lds_void*)((char*)g_poll_raw + i * 1024), 16, 0, kPolDev);
      __builtin_amdgcn_s_waitcnt(0);
      bool ok = true;
      const lds_u32x4* rq = (const lds_u32x4*)(lds_void*)g_poll_raw;
      for (int i = 2 * lane; i < n; i += 128) {
        const u32x4 q = rq[i >> 1];
        ok &= q.y == e && q.w == e;
        const int o = SW ? xsw(i) : i;  // i even: i + 1 lands at o + 1
        dst[o] = __uint_as_float(q.x);
        dst[o + 1] = __uint_as_float(q.z);
      }
      if (__all(ok)) return true;
    }
    if ((spin & 63) == 63) {
      if (ld_u32_dev(ws, Ws::kErr) != 0) return false;
      if (spin > kSpinLimit) {
        if (lane == 0) fail(c, code, f, l);
        return false;
      }
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

constexpr int kH = 2048, kI = 6144;
template <>
struct SpreadLate<kH, kI> {
  static constexpr bool value = true;
};
// the sampled pick with half the value registers in flight: the 168-register budget of 9 waves
template <>
struct PickBatch<kTalkerV, kTalkerV / kWG> {
  static constexpr int value = 4;
};
static_assert(sizeof(Lds<kH, kI, 8, kTalkerV, false>) + sizeof(g_poll_raw) + 64 <= 160 * 1024, "LDS over 160 KB");
static_assert(kI <= kRawCells && kH <= kRawCells && kQ <= kRawCells, "poll staging too small");

// The polls of the 1.7B control wave, by the (MAXB, SW) pair poll_cells is instantiated with:
//   <mb(512), false>: q | k | v of one kv head, 32 rows of 16 cells, each row published by one workgroup (probed);
//   <mb(H), false>: o projection or down projection output, H / 256 cells per workgroup (read whole);
//   <mb(I), true> with n = I: gate/up activation, I / 256 cells per workgroup (probed);
//   <mb(kQ), true> with n = kQ: attention output, 4 cells per merging lane group (read whole).
static_assert(mb(512) == 4 && mb(kH) == 16 && mb(kI) == 16 && mb(kQ) == 16, "poll instantiations moved");
template <>
__device__ bool poll_cells<4, false>(const void* cells, uint32_t idx0, int n, uint32_t e, float* dst, void* ws,
                                     int lane, const Ctx& c, uint32_t code, int f, int l) {
  return poll_cells_lds<false>(cells, idx0, n, 16, e, dst, ws, lane, c, code, f, l);
}
template <>
__device__ bool poll_cells<16, false>(const void* cells, uint32_t idx0, int n, uint32_t e, float* dst, void* ws,
                                      int lane, const Ctx& c, uint32_t code, int f, int l) {
  return poll_cells_lds<false, false>(cells, idx0, n, n / kWG, e, dst, ws, lane, c, code, f, l);
}
template <>
__device__ bool poll_cells<16, true>(const void* cells, uint32_t idx0, int n, uint32_t e, float* dst, void* ws,
                                     int lane, const Ctx& c, uint32_t code, int f, int l) {
  if (n == kQ) return poll_cells_lds<true, false>(cells, idx0, n, 4, e, dst, ws, lane, c, code, f, l);
  // gate/up activation: the probe looks at the last cell of every fourth producer (64 probes, one per lane);
  // the read still checks every cell (measured: 1% faster than probing all 256)
  return poll_cells_lds<true>(cells, idx0, n, 4 * (n / kWG), e, dst, ws, lane, c, code, f, l);
}

}  // namespace

int sk_talker_frames_2048(const sk_talker_desc* d, int n_frames, hipStream_t st) {
  const CpArgs none{};
  return launch_frames<kH, kI, 8, kTalkerV, false>(d, none, n_frames, st);
}
