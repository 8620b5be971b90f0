// sk_frames_place: measures, for a frame-kernel workspace, which page of the periods of each 512 KB quarter of its cell
// region is nearest each XCD, and records the page slot of every XCD's copy of the cells in the workspace
// (Ws::kPlace, one word per quarter).
//
// Each 4 KB page of HBM is served from one place on the chip; a device-coherent store becomes visible to loads from
// the XCD nearest that place about 0.42 us after it is issued, and to the farthest XCD about 0.69 us after. Within a
// 512 KB quarter of a 2 MB-aligned region the same page slot of every 32 KB period is nearest the same XCD (eight
// slots, each nearest a different XCD); the quarters differ. The measurement is a schedule of rounds on the 100 MHz
// clock every workgroup shares: in each round one workgroup stores a new value into one page and every other
// workgroup times how long the value takes to reach it. Per quarter, the eight pages of its first and of its last
// period are measured from two producers each and assigned to the XCDs (nearest first), and both periods must agree
// with the assignment. It runs once per workspace (the frame kernels read the result at every launch); a quarter whose
// measurement is not consistent, or a workspace never measured or zeroed since, uses the fixed placement (XCD x's
// copy in page x): the same results, slower exchanges.
#include "frame_impl.h"

#include <atomic>

namespace {

// rounds: per quarter, the 8 pages of its first and of its last period, each from two producers
constexpr int kRoundsPerQuarter = 2 * 8 * 2;
constexpr int kPlaceRounds = kQuarters * kRoundsPerQuarter;  // 128
constexpr uint32_t kRoundTicks = 500;                        // 5 us per round
constexpr uint32_t kLeadTicks = 100;                         // consumers start polling 1 us early
constexpr int kPlacePolls = 4096;                            // loads per consumer and round, at most
constexpr uint32_t kPlaceByte = 64;                          // the word written: cell 8's value (its epoch stays)
constexpr float kPlaceTol = 8.f;                             // ticks (80 ns): pages of the XCD's own pair pass
constexpr uint32_t kNone = 0xffffffffu;
// The latencies [round][workgroup] (u32 ticks; kNone: the producer, or no value seen), then the means
// [quarter][first / last period][page][XCD] (f32); in the trace area.
constexpr uint32_t kTableBytes = (uint32_t)kPlaceRounds * kWG * 4, kMeansBytes = kQuarters * 2 * 64 * 4;
static_assert(kTableBytes + kMeansBytes <= Ws::kTraceBytes, "table fits");

// round r: quarter, period (first or last of the quarter), page and producer XCD
struct Round {
  int q, last, page, prod;
};
__device__ __forceinline__ Round round_of(int r) {
  const int q = r / kRoundsPerQuarter, k = r % kRoundsPerQuarter, last = k >> 4, j = k & 15;
  return {q, last, j >> 1, ((j >> 1) + 4 * (j & 1) + last) & 7};
}
__device__ __forceinline__ uint64_t rt_now() {
  const uint64_t t = __builtin_amdgcn_s_memrealtime();
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  return t;
}

__global__ __launch_bounds__(64) void k_place(void* ws, uint32_t nonce) {
  const int lane = threadIdx.x;
  __shared__ int s_g;
  __shared__ float s_avg[kQuarters][2][8][8];
  __shared__ uint32_t s_lat[kPlaceRounds];  // this workgroup's latencies (LDS: no store in flight during the rounds)
  char* region = cell_region(ws);
  uint32_t* table = (uint32_t*)((char*)ws + Ws::kTrace);
  float* means = (float*)((char*)ws + Ws::kTrace + kTableBytes);
  if (lane == 0) {
    const uint32_t x = xcc_id();
    const uint32_t rk = __hip_atomic_fetch_add((uint32_t*)((char*)ws + Ws::kPlaceArrive + 4 * (x & 7)), 1u,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t all = __hip_atomic_fetch_add((uint32_t*)((char*)ws + Ws::kPlaceAll), 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    uint64_t* t0p = (uint64_t*)((char*)ws + Ws::kPlaceT0);
    if (all == kWG - 1) __hip_atomic_store(t0p, rt_now() + 2000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint64_t T0 = 0;
    for (int s = 0; s < (1 << 22) && T0 == 0; s++) {
      T0 = __hip_atomic_load(t0p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (T0 == 0) __builtin_amdgcn_s_sleep(2);
    }
    const bool placed = x < (uint32_t)kXcd && rk < (uint32_t)kPerXcd && T0 != 0;
    const int g = placed ? (int)(x * kPerXcd + rk) : -1;
    s_g = g;
    if (placed) {
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(region);
      uint32_t sink = 0;
      for (int r = 0; r < kPlaceRounds; r++) {
        const Round rd = round_of(r);
        const uint32_t period = 16u * (uint32_t)rd.q + (rd.last ? 15u : 0u);
        const uint32_t off = period * 32768u + (uint32_t)rd.page * 4096u + kPlaceByte;
        const uint32_t tag = (nonce << 8) | (uint32_t)r;
        const uint64_t S = T0 + (uint64_t)r * kRoundTicks;
        uint32_t lat = kNone;
        if (x == (uint32_t)rd.prod && rk == 0) {
          for (int s = 0; s < (1 << 24) && rt_now() < S; s++) {}
          __builtin_amdgcn_raw_buffer_store_b32(tag, rs, off, 0, kPolDev);
        } else {
          for (int s = 0; s < (1 << 24) && rt_now() + kLeadTicks < S; s++) {}
          for (int p = 0; p < kPlacePolls; p++) {
            const uint32_t v = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, kPolDev);
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            sink += v;
            if (v == tag) {
              const uint64_t t = rt_now();
              lat = t > S ? (uint32_t)(t - S) : 0u;
              break;
            }
          }
        }
        s_lat[r] = lat;
      }
      if (sink == 0x9e3779b9u) st_u32_dev(ws, Ws::kPlaceSink, sink);  // keeps the loads' values live
    }
  }
  __syncthreads();
  // end of the rounds: every workgroup's latencies are stored before workgroup 0 reads them (bounded wait)
  if (s_g >= 0)
    for (int r = lane; r < kPlaceRounds; r += 64) st_u32_dev(table, (uint32_t)(r * kWG + s_g) * 4u, s_lat[r]);
  __builtin_amdgcn_s_waitcnt(0);
  if (lane == 0)
    __hip_atomic_fetch_add((uint32_t*)((char*)ws + Ws::kPlaceEnd), 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  if (s_g != 0) return;
  bool all_in = false;
  for (int s = 0; s < (1 << 22); s++) {
    if (ld_u32_dev(ws, Ws::kPlaceEnd) >= (uint32_t)kWG) { all_in = true; break; }
    __builtin_amdgcn_s_sleep(2);
  }
  // lane = page * 8 + XCD: the mean latency of that XCD's workgroups over the page's rounds, per quarter and period
  const int page = lane >> 3, xx = lane & 7;
  for (int q = 0; q < kQuarters; q++)
    for (int last = 0; last < 2; last++) {
      float sum = 0.f;
      int n = 0;
      for (int pi = 0; pi < 2; pi++) {
        const int r = q * kRoundsPerQuarter + last * 16 + page * 2 + pi;
        for (int w = 0; w < kPerXcd; w++) {
          const uint32_t v = ld_u32_dev(table, (uint32_t)(r * kWG + xx * kPerXcd + w) * 4u);
          if (v != kNone) { sum += (float)v; n++; }
        }
      }
      const float m = n > 0 ? sum / (float)n : 1e30f;
      s_avg[q][last][page][xx] = m;
      st_u32_dev(means, (uint32_t)((q * 2 + last) * 64 + lane) * 4u, __float_as_uint(m));
    }
  __syncthreads();
  if (lane < kQuarters) {
    // lane q: the quarter's pages assigned nearest first (the smallest latency, summed over the quarter's first and
    // last period, among free pages and XCDs, eight times); kept when every XCD's page is within 80 ns of its
    // nearest in both periods (the two XCDs of a pair differ by less than that, the other pairs by more)
    const int q = lane;
    uint32_t slot[8] = {}, page_used = 0, x_done = 0;
    bool ok = all_in;
    for (int it = 0; it < 8; it++) {
      float best = 1e31f;
      int bp = 0, bx = 0;
      for (int p = 0; p < 8; p++)
        for (int c = 0; c < 8; c++) {
          const float v = s_avg[q][0][p][c] + s_avg[q][1][p][c];
          if (!(page_used >> p & 1) && !(x_done >> c & 1) && v < best) { best = v; bp = p; bx = c; }
        }
      ok = ok && best < 1e29f;
      slot[bx] = (uint32_t)bp;
      page_used |= 1u << bp;
      x_done |= 1u << bx;
    }
    uint32_t w = 0;
    for (int c = 0; c < 8; c++) {
      for (int last = 0; last < 2; last++) {
        float mn = s_avg[q][last][0][c];
        for (int p = 1; p < 8; p++) mn = fminf(mn, s_avg[q][last][p][c]);
        ok = ok && s_avg[q][last][slot[c] & 7][c] <= mn + kPlaceTol;
      }
      w |= (slot[c] & 7u) << (3 * c);
    }
    st_u32_dev(ws, Ws::kPlace + 4u * (uint32_t)q, ok ? (w | 0x80000000u) : 0u);
  }
}

}  // namespace

extern "C" int sk_frames_place(void* workspace, int64_t workspace_bytes, void* stream) {
  if (!workspace) return sk_set_error(SK_EINVAL, "sk_frames_place: null workspace");
  if (workspace_bytes < Ws::kBytes) return sk_set_error(SK_EWORKSPACE, "sk_frames_place: workspace too small");
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return sk_check_launch(e, "sk_frames_place: no current HIP device");
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return sk_check_launch(e, "sk_frames_place: reading the CU count");
  if (cus != kWG) return sk_set_error(SK_EUNSUPPORTED, "sk_frames_place: needs a 256-CU device (8 XCDs x 32)");
  static std::atomic<uint32_t> calls{0};
  const uint32_t nonce = (calls.fetch_add(1u) % 0xfffffeu) + 1u;  // 24 bits, never 0: each call's values are new
  hipStream_t st = (hipStream_t)stream;
  e = hipMemsetAsync((char*)workspace + Ws::kPlaceArrive, 0, Ws::kPlaceT0 + 8 - Ws::kPlaceArrive, st);
  if (e != hipSuccess) return sk_check_launch(e, "sk_frames_place: clearing its counters");
  hipLaunchKernelGGL(k_place, dim3(kWG), dim3(64), 0, st, workspace, nonce);
  return sk_check_launch(hipGetLastError(), "sk_frames_place");
}
