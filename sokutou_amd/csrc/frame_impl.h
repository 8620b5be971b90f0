#pragma once
// Persistent talker decode kernel (device code and launch templates; the entry points are in frame.hip for the
// talker and frame_cp.hip for the code predictor, separate translation units so that the code generated for one
// mode does not depend on the other's): whole frames (28 layers + final norm + codec head + greedy pick + next
// embedding) in one launch of 256 workgroups, one per CU.
//
// It computes what the five per-layer launches of the reference compute (qwen3/kernels.py:619-627, frame order
// 676-685, with `embed` feeding the next token as in qwen3/kernels.py:642), but as a dataflow over the whole chip:
//
//  * XCD-aware placement. The talker has 8 kv heads and MI355X has 8 XCDs: kv head x is owned by the 32 workgroups
//    of XCD x. Each workgroup learns its XCD from the hardware XCC_ID register and a dense rank 0..31 from an
//    arrival counter (the block -> XCD assignment is round-robin with a start that moves between dispatches).
//  * Stages of a layer, each a set of rows of one projection per workgroup:
//      S1 qkv     rows of head x (q of heads 2x, 2x+1, k and v of head x), 16 per workgroup
//      S2 attn    positions [t0, t1) of head x (the cache length split 32 ways), both q heads; unnormalised
//                 partial (m, l, o) per workgroup; the owner of `pos` appends K/V to the cache
//      S3 merge   dims [8r, 8r+8) of heads 2x, 2x+1: log-sum-exp merge of the 32 partials
//      S4 o       H/256 rows of the output projection, added to the residual
//      S5 gu      2I/256 interleaved gate/up rows with RMSNorm, silu(g)*u
//      S6 down    H/256 rows of the down projection, added to the residual
//    then per frame: head rows (with the talker processor) and a local argmax, and every workgroup reduces the
//    256 candidates itself and loads the next embedding row.
//  * Exchanges use 8-byte cells {value, epoch} written and read with device-coherent (sc1) accesses: a consumer
//    polls the cells it needs until all carry the producer's epoch. A 64-bit aligned store is single-copy atomic,
//    so data and readiness arrive together and no fence, flag or L2 writeback is needed.
//  * Wave roles. Waves 0..3 compute; wave 4 (the control wave) does all polling and copies inputs into LDS.
//    The compute waves issue only weight and K/V loads: as soon as a stage's registers are consumed, the same
//    registers are reloaded with that stage's weights of the next layer, so the HBM stream runs a full layer
//    ahead of the dependency chain. The hardware waits for loads in issue order per wave, which is why polling
//    (whose completion time is unknown) lives in a wave that has no prefetches queued.
//  * Every wait is bounded. A timeout or an inconsistent placement sets an error word in the workspace; every
//    poll also watches that word, so all workgroups leave promptly and the host reports the error.
//
// Numerics are those of the per-op kernels: fp32 residual and accumulation, bf16 K/V cache written round to
// nearest even, per-row bf16 weight scales applied after the dot, RMSNorm scale applied after the dot.
#include <type_traits>

#include "common.h"
#include "internal.h"

namespace {

constexpr int kXcd = 8, kPerXcd = 32, kWG = kXcd * kPerXcd;
constexpr int kChunks = kPerXcd;           // attention split of the cache length per head
constexpr int kNQ = 16, kNKV = 8, kQKV = (kNQ + 2 * kNKV) * SK_HD, kQ = kNQ * SK_HD;
constexpr int kTalkerV = 3072;             // talker codec vocabulary
constexpr uint32_t kSpinLimit = 1u << 19;
constexpr float kInvSqrtHd = 0.08838834764831845f;
constexpr int kNT = 2;  // buffer cache policy bit nt (non-temporal): the streamed weights

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t xcc_id() { return __builtin_amdgcn_s_getreg((20) | (0 << 6) | (15 << 11)) & 0xfu; }
// lane i's 64-bit value, wave-uniform (i wave-uniform)
__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int i) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), i) << 32) |
         (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, i);
}

// ---- exchange cells ------------------------------------------------------------------------------------------
// The cells live in a 2 MB region of the workspace, aligned to 2 MB. Cell i of the index space (Layout) lies in
// block i / 512 (512 cells, one 4 KB page); block b owns period b of the region (32 KB, 8 pages), and each XCD has a
// copy of the block in one page of the period. Each 4 KB page of HBM is served from one place on the chip, about
// 0.42 us of device-coherent store-to-load latency away from the XCD nearest to it and up to 0.69 us from the
// farthest, and within a 512 KB quarter of the region the same page of every period is nearest the same XCD;
// sk_frames_place measures which. XCD x reads its copy from its nearest page of each quarter (`slots`: 3 bits per
// quarter), the producer of a cell that every XCD reads stores all eight pages of the period (the *_all stores),
// and the cells of an exchange inside one XCD (q|k|v and the attention partials of its head pair) exist in that
// XCD's page only, so local index ranges serve all eight XCDs at once.
constexpr uint32_t kRegionBytes = 2u << 20, kRegionCells = 64u * 512u;  // 64 periods of 8 pages
constexpr int kQuarters = 4;                                             // 16 periods each
__host__ __device__ constexpr uint32_t cell_off(uint32_t i) { return ((i >> 9) << 15) | ((i & 511u) << 3); }
// byte offset of cell i in the copy of the XCD whose page slots are `slots`
__host__ __device__ constexpr uint32_t own_off(uint32_t slots, uint32_t i) {
  return cell_off(i) | (((slots >> (3u * (i >> 13))) & 7u) << 12);
}
// byte offset of cell i of a range every XCD reads, in the kernels that keep one copy of it (SINGLE: the hidden-2048
// i8g32 and bf16 kernels): block b in page b % 8 of its period, so an exchange's consecutive blocks lie in different
// pages, as a plain array's would
__host__ __device__ constexpr uint32_t single_off(uint32_t i) { return cell_off(i) | (((i >> 9) & 7u) << 12); }
template <bool SINGLE>
__host__ __device__ constexpr uint32_t read_off(uint32_t slots, uint32_t i) { return SINGLE ? single_off(i) : own_off(slots, i); }

// Accesses of this XCD's copy (`region` the cell region, `slots` this XCD's page slots).
__device__ __forceinline__ void put(void* region, uint32_t slots, uint32_t idx, float v, uint32_t e) {
  u32x2 x = {__float_as_uint(v), e};
  __builtin_amdgcn_raw_buffer_store_b64(x, make_rsrc(region), own_off(slots, idx), 0, kPolDev);
}
template <bool SINGLE = false>
__device__ __forceinline__ u32x4 get2(const void* region, uint32_t slots, uint32_t idx) {  // cells idx, idx+1
  return __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(region), read_off<SINGLE>(slots, idx), 0, kPolDev);
}
// cells idx + 2 lane, + 1 with idx wave-uniform and a multiple of 128 (so the 128 cells lie in one block): the lane
// part goes in the one vector offset every such load shares (16 lane bytes), the uniform part in the scalar offset,
// so a poll of many loads holds one address register.
template <bool SINGLE = false>
__device__ __forceinline__ u32x4 get2l(const void* region, uint32_t slots, uint32_t idx, int lane) {
  return __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(region), (uint32_t)lane * 16u,
                                               __builtin_amdgcn_readfirstlane(read_off<SINGLE>(slots, idx)), kPolDev);
}
// The same cells with a vector address per load (the hidden-1024 kernels' polls).
template <bool SINGLE = false>
__device__ __forceinline__ u32x4 get2v(const void* region, uint32_t slots, uint32_t idx, int lane) {
  return __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(region), read_off<SINGLE>(slots, idx) + (uint32_t)lane * 16u, 0,
                                               kPolDev);
}
// cell idx + vbytes / 8 (vbytes per lane) of this XCD's copy, with the cells of the wave inside idx's block
__device__ __forceinline__ void putl(void* region, uint32_t slots, uint32_t idx, uint32_t vbytes, float v, uint32_t e) {
  u32x2 x = {__float_as_uint(v), e};
  __builtin_amdgcn_raw_buffer_store_b64(x, make_rsrc(region), vbytes, __builtin_amdgcn_readfirstlane(own_off(slots, idx)),
                                        kPolDev);
}
// Stores of a cell every XCD reads, into all eight pages of its period at vector offset vo (the cell's place in the
// first page): one address register stepped by a page after each store (eight scalar page offsets, or eight vector
// addresses formed up front, made the kernels spill more).
template <class T>
__device__ __forceinline__ void store_pages(void* region, uint32_t vo, const T& x) {
#pragma unroll
  for (int pg = 0; pg < 8; pg++) {
    if constexpr (sizeof(T) == 16) __builtin_amdgcn_raw_buffer_store_b128(x, make_rsrc(region), vo, 0, kPolDev);
    else __builtin_amdgcn_raw_buffer_store_b64(x, make_rsrc(region), vo, 0, kPolDev);
    vo += 4096u;
    __asm__ volatile("" : "+v"(vo));
  }
}
// (SINGLE: the one copy)
template <bool SINGLE = false>
__device__ __forceinline__ void put_all(void* region, uint32_t idx, float v, uint32_t e) {
  const u32x2 x = {__float_as_uint(v), e};
  if constexpr (SINGLE) __builtin_amdgcn_raw_buffer_store_b64(x, make_rsrc(region), single_off(idx), 0, kPolDev);
  else store_pages(region, cell_off(idx), x);
}
template <bool SINGLE = false>
__device__ __forceinline__ void put2_all(void* region, uint32_t idx, float v0, float v1, uint32_t e) {
  const u32x4 x = {__float_as_uint(v0), e, __float_as_uint(v1), e};
  if constexpr (SINGLE) __builtin_amdgcn_raw_buffer_store_b128(x, make_rsrc(region), single_off(idx), 0, kPolDev);
  else store_pages(region, cell_off(idx), x);
}
// Cells idx, idx + 1 (values wave-uniform) into all eight pages, lane k < 8 storing page k (SINGLE: lane 0, the one
// copy).
template <bool SINGLE = false>
__device__ __forceinline__ void put2_lanes(void* region, uint32_t idx, float v0, float v1, uint32_t e, int lane) {
  if (lane < (SINGLE ? 1 : 8)) {
    u32x4 x = {__float_as_uint(v0), e, __float_as_uint(v1), e};
    __builtin_amdgcn_raw_buffer_store_b128(x, make_rsrc(region), SINGLE ? single_off(idx) : ((uint32_t)lane << 12) + cell_off(idx),
                                           0, kPolDev);
  }
}
__device__ __forceinline__ uint32_t ld_u32_dev(const void* base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(base), off, 0, kPolDev);
}
__device__ __forceinline__ void st_u32_dev(void* base, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, make_rsrc(base), off, 0, kPolDev);
}

// Workgroup barrier that does not wait for outstanding global loads (the compute waves keep their weight
// prefetches in flight across it); it only makes this wave's LDS writes visible first.
__device__ __forceinline__ void wg_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt/expcnt untouched
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- layout of the workspace (bytes) -------------------------------------------------------------------------
struct Ws {
  // control words
  static constexpr uint32_t kErr = 0, kTick = 4, kLaunch = 8, kDiag = 16, kTraceOn = 32, kPollDelay = 40,
                            kPlace = 48, kCensus = 64;  // place: 4 words; census: 8 counters
  // kPlace: the cell placement sk_frames_place measured, one word per quarter of the cell region (bits 0-23: the
  // page slot of each XCD's copy, 3 bits per XCD; bit 31: set by a measurement); a quarter without a measurement
  // uses the fixed placement, XCD x's copy in page x.
  // Polling of a stage's input starts this many sleep units (s_sleep 1: 64 shader clocks, ~27 ns at 2.4 GHz)
  // after the workgroup published its own part of it. Reads that reach the cells before the producers' stores
  // are visible come back stale and make the whole exchange slower than one late, successful read. One delay
  // per exchange (kHop*), since producers and timing differ: bytes kPollDelay + h of the workspace override
  // the defaults (value - 1) when non-zero.
  static constexpr int kHopS1 = 0, kHopS2 = 1, kHopS3 = 2, kHopS4 = 3, kHopS5 = 4, kHopS6 = 5, kHopHead = 6,
                       kHopPick = 7, kHops = 8;
  // sk_frames_place's own words: arrivals per XCD [8], arrivals, its end barrier, the start time (8 bytes), a sink
  static constexpr uint32_t kPlaceArrive = 96, kPlaceAll = 128, kPlaceEnd = 132, kPlaceT0 = 136, kPlaceSink = 144;
  static constexpr int kTraceLayers = 32, kTraceEvents = 16;  // optional per-stage timestamps of frame 0
  // trace stamps [256 workgroups][2 roles][32 layers][16 events] of 8 bytes (sk_frames_place's latency table while
  // it runs), then the cell region: the first 2 MB boundary at or after kRegionMin
  static constexpr uint32_t kTrace = 256, kTraceBytes = (uint32_t)kWG * 2u * kTraceLayers * kTraceEvents * 8u;
  static constexpr uint32_t kRegionMin = kTrace + kTraceBytes;
  static constexpr int64_t kBytes = (int64_t)kRegionMin + 2 * (int64_t)kRegionBytes;
};
// the cell region of workspace ws
__host__ __device__ inline char* cell_region(void* ws) {
  return (char*)(((uintptr_t)ws + Ws::kRegionMin + kRegionBytes - 1) & ~(uintptr_t)(kRegionBytes - 1));
}

// The index space of the cells (Layout). Local ranges first (each XCD's own copy; every range starts on a block):
//   e1  q|k|v of the XCD's head pair [512]
//   e2m the attention partials' softmax statistics [32 chunks][m0 l0 m1 l1]
//   e2o the partials' outputs [32 chunks][2 heads][128]
//   b1  the code predictor's paired pass: the second row's q|k|v [512]
// then the ranges every XCD reads (all copies written):
//   e3 attention output [2048], e4 h after o [H], e5 activation [I], e6 h after down [H], e7 pick candidates
//   [256][2] (greedy) or maxima [256] (sampled), e8 processed logits of a sampled pick [vocab <= 3072], and for the
//   code predictor the paired pass's second row (b3 attention output, b4 h after o, b5 activation, b6 h after down)
//   and the projected input pj [H]. The talker's kernels use the cells up to e8's end.
struct Layout {
  uint32_t e1 = 0, e2m = 0, e2o = 0, b1 = 0, e3 = 0, e4 = 0, e5 = 0, e6 = 0, e7 = 0, e8 = 0, b3 = 0, b4 = 0, b5 = 0,
           b6 = 0, pj = 0, talker_end = 0, total = 0;
  __host__ __device__ constexpr Layout(int H, int I) {
    e1 = 0;
    e2m = 512;
    e2o = 1024;
    b1 = e2o + (uint32_t)kChunks * 2u * SK_HD;
    e3 = b1 + 512;
    e4 = e3 + kQ;
    e5 = e4 + H;
    e6 = e5 + I;
    e7 = e6 + H;
    e8 = e7 + 512;
    talker_end = e8 + kTalkerV;
    b3 = talker_end;
    b4 = b3 + kQ;
    b5 = b4 + H;
    b6 = b5 + I;
    pj = b6 + H;
    total = pj + H;
  }
};
// Every range starts on a block at the shapes built (H and I multiples of 512), the talker's cells fit the region
// at both shapes, and the code predictor's (hidden 1024) too.
static_assert(Layout(1024, 3072).total <= kRegionCells && Layout(2048, 6144).talker_end <= kRegionCells, "cells fit");
static_assert(Layout(2048, 6144).e5 % 512 == 0 && Layout(1024, 3072).b6 % 512 == 0 && Layout(1024, 3072).e2o % 512 == 0,
              "ranges start on a block");
static_assert((uint32_t)kChunks * 4u <= 512u && (2u * SK_HD) * 2u == 512u, "two chunks' outputs per block");

}  // namespace

// Descriptor layouts shared with the host (declared in sokutou_amd.h).
static_assert(sizeof(sk_layer_desc) == 14 * sizeof(void*), "sk_layer_desc layout");

namespace {

// Order-preserving key of (value, index): larger value wins, then the lower index.
__device__ __forceinline__ uint64_t pick_key(float v, int i) {
  const uint32_t u = __float_as_uint(v);
  const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((uint64_t)k << 32) | (uint32_t)(0xffffffffu - (uint32_t)i);
}

// Spread late prefetch: o after the attention, gate/up after o, down after gate/up, the next layer's qkv and K/V
// after down. Each stage's weights are then in flight across exactly one exchange, and
// the registers they occupy are live from one stage to the next only. Off unless a translation unit specialises
// it for its shape before instantiating the kernel.
template <int H, int I>
struct SpreadLate {
  static constexpr bool value = false;
};
// Global addressing of a shape's kernel: true = the lane part of every cell, weight-row and cache address in one
// shared vector offset (lane bytes) and the wave-uniform part in the scalar offset of buffer instructions
// (get2l, putl, weight rows by row start); false = a vector address per load or store. The hidden-2048
// kernel (frame17.hip) takes the shared offsets: with a vector address per load its waves spilled the addresses
// (per-row weight pointers, poll and publish offsets) and reloaded them from scratch on every exchange. The
// hidden-1024 kernels keep per-load addresses, the code they were tuned with (measured 4% slower with get2l polls).
template <int H>
struct LaneOffsetPolls {
  static constexpr bool value = false;
};
// With kSpread: the first half of each wave's gate/up rows is loaded with o, after the attention (two exchanges
// before their use), the second half one exchange before, as kSpread loads them all. The hidden-2048 gate/up
// rows stream 25 MB per layer, more than one exchange can hide. Off unless a translation unit specialises it.
template <int H, int I>
struct SplitGateUp {
  static constexpr bool value = false;
};
// Width of the code predictor's input before its projection (small_to_mtp_projection, qwen3/kernels.py:520-521,
// 629-637): 0, no projection (the position inputs are H wide and enter the stack as they are). A translation unit
// specialises it before instantiating the code-predictor kernels of a projected code predictor (the 1.7B
// Qwen3-TTS: 2048-wide inputs into a 1024-wide stack); each position then starts with a projection stage.
template <int H, int I>
struct CpProjIn {
  static constexpr int value = 0;
};

// W, the compute waves per workgroup, is 4: one per SIMD, with the control wave as the fifth wave of the CU. Each
// wave then has 256 registers, which is what lets a whole layer of hidden-1024 weights sit in registers and the
// control wave poll every exchange into registers.
template <int H, int I, int W, int V, bool CP>
struct Cfg {
  static_assert(W == 4, "four compute waves");
  static constexpr int R_O = H / kWG, R_GU = 2 * I / kWG, R_D = H / kWG;
  static constexpr int RW_QKV = 16 / W;                       // rows per compute wave
  static constexpr int RW_O = (R_O + W - 1) / W, RW_GU = R_GU / W, RW_D = (R_D + W - 1) / W;
  static constexpr int kHeadRows = V / kWG;                   // head rows per workgroup: 12 (talker), 8 (code predictor)
  static constexpr int RW_HEAD = (kHeadRows + W - 1) / W;
  static constexpr int CH = H / 1024, CQ = kQ / 1024, CI = I / 1024;  // 16-byte chunks per lane per row
  static constexpr int KVL = H > 1024 ? 4 : 2;                 // K (and V) loads per lane
  static constexpr int kMaxChunk = 4 * W * KVL;                // positions per attention workgroup: 32 / 64
  static constexpr int kMaxLen = kMaxChunk * kChunks;          // 1024 / 2048
  // Prefetch distances. At hidden 1024 every stage's weights for the next layer are held in registers (a full
  // layer ahead). A full layer of 1.7B weights does not fit beside the rest (192 registers per wave); each stage's
  // weights are then loaded one to three exchanges before their use (kLate): o and gate/up after the attention of
  // their layer, down and the next layer's qkv after gate/up. kSpread (SpreadLate) moves them later still, one
  // exchange before their use.
  static constexpr bool kLate = H > 1024;
  static constexpr bool kSpread = kLate && SpreadLate<H, I>::value;
  // code-predictor caches short enough for one workgroup to attend over all of them (see Chunk::whole)
  static __device__ bool whole(int pos) { return CP && pos + 1 <= kMaxChunk; }
  static_assert(16 % W == 0 && R_GU % W == 0 && R_GU % 2 == 0, "row split");
};
// The compute waves' view of Cfg for weight format WD. bf16 weights take two 16-byte loads per 16-weight chunk
// (CH, CQ, CI count loads per lane and row), twice the registers of int8; their stages are loaded one exchange
// before their use (kLate, kSpread) instead of a whole layer ahead, whatever the shape does for int8.
template <int H, int I, int W, int V, bool CP, int WD>
struct CfgW : Cfg<H, I, W, V, CP> {
  using B = Cfg<H, I, W, V, CP>;
  static constexpr int WB = WD == SK_WD_BF16 ? 2 : 1;
  static constexpr int CH = B::CH * WB, CQ = B::CQ * WB, CI = B::CI * WB;
  static constexpr bool kLate = B::kLate || WD == SK_WD_BF16;
  static constexpr bool kSpread = B::kSpread || WD == SK_WD_BF16;
  // One copy of every cell that all XCDs read (single_off) instead of one per XCD: the hidden-2048 i8g32 and bf16
  // kernels, whose registers are full (bf16 weights one exchange ahead). Their copies cost more than their nearer
  // reads gained: 1004 against 943 us per frame (bf16) and 672 against 659 (i8g32) with eight copies, while the
  // i8row kernel at that shape broke even (637) and the hidden-1024 ones gained 4-7%.
  static constexpr bool kSingle = H > 1024 && WD != SK_WD_I8ROW;
};

// floats of a GEMV staging buffer for n elements (n a multiple of 64): one 8-byte slot of padding after every 32
// (xsw, below)
constexpr int xs_floats(int n) { return n + n / 32; }

// LDS of the frame kernel
template <int H, int I, int W, int V, bool CP>
struct Lds {
  static constexpr int XS = I > kQ ? I : kQ;
  float hin[H];        // residual entering the layer (S1; read back by S4), or the final residual (head)
  float hmid[H];       // residual after the o projection (S5; read back by S6)
  float xs[2][xs_floats(XS)];  // staged GEMV inputs (xsw), alternating so the control wave can fill the next stage's input
                       // while the compute waves still read the current one: [0] S1/S5/head, [1] S4/S6
  float qkv[512];      // S2: q0 | q1 | k | v of this workgroup's head
  float qs[2][SK_HD];  // normalised, rotated, scaled q
  float kn[SK_HD], vn[SK_HD];
  float sc[2][Cfg<H, I, W, V, CP>::kMaxChunk];
  float pub[64];           // this workgroup's outputs of a stage, published by the last compute wave to finish
  uint32_t pubcnt;         // compute-wave arrivals at publish (counts up; the wave that makes it a multiple of W
                           // publishes)
  float inv;
  sk_layer_desc desc[Ws::kTraceLayers];  // the layer descriptors, copied once per launch
  uint64_t cand[W];
  float hv[16];        // this workgroup's processed logits (sampled picks)
  int flags[8];
  int64_t tok;
  uint32_t pubseq;  // stage publications completed by the compute waves
};

// The second row of the code predictor's paired first pass (positions 0 and 1 together): its residuals, staged
// GEMV inputs, q|k|v and attention vectors. Placed after Lds in the code-predictor kernels' LDS only.
template <int H, int I>
struct LdsPair {
  static constexpr int XS = I > kQ ? I : kQ;
  float hin[H], hmid[H];
  float xs[2][xs_floats(XS)];
  float qkv[512];
  float qs[2][SK_HD];
  float kn[SK_HD], vn[SK_HD];
  float red[8];
  float inv;
  int bad;  // a compute wave's poll of the second row failed (cleared at the start of the pass)
};
// Byte offset of the sampled pick's LDS copy of the value cells (V x 8 bytes, 16-byte aligned), after Lds; only the
// sampling instantiations allocate it.
template <int H, int I, int W, int V, bool CP>
constexpr size_t kPickCopy = (sizeof(Lds<H, I, W, V, CP>) + 15) / 16 * 16;


// Records a timeout: error code, then frame and layer of the stage that gave up (diagnostic words of the workspace).
struct Ctx;
__device__ void fail(const Ctx& c, uint32_t code, int f, int l);

// GEMV inputs are staged in LDS in 8-byte slots, one per element pair. Lane L of a dot multiplies byte 4 j + t of
// its weight chunk c with element 16 (L + 64 c) + 4 j + t, and reads those 4 elements as the pairs
// P = 8 (L + 64 c) + 2 j + h (h = 0, 1) with two 8-byte reads; the control wave stages the pairs P = L + 64 b. Pair P
// sits in slot P + P / 32 (one slot of padding after every 32): across the 32 lanes of a half-wave both patterns then
// reach 32 different bank pairs (unpadded, the dot's reads fell 64 bytes apart, two lanes per bank pair, and the
// staging writes four; SQ_LDS_BANK_CONFLICT on the 0.6B talker: 9.1e8 cycles per launch unpadded, 6.7e8 padded;
// the frame rate is the same, the conflicts were off the critical path), and each lane's slot stays its own base
// plus a compile-time offset (a XOR swizzle, also conflict-free, made the offsets per lane and spilled 9-35
// registers). A vector staged at an
// element offset that is a multiple of 64 starts at xsw(offset). 8-byte rather than 16-byte reads: 16-byte LDS
// reads of the same data stall the LDS on gfx950 (SQ_LDS_UNALIGNED_STALL; 2250 against 820 cycles per stage).
__device__ __forceinline__ int xslot(int P) { return P + (P >> 5); }
// float index of element i (i even: i + 1 lands at xsw(i) + 1)
__device__ __forceinline__ int xsw(int i) { return 2 * xslot(i >> 1) + (i & 1); }
// 8-byte slot of the dot's read h of quarter q = 4 c + j (chunk c, bytes 4 j .. 4 j + 3) for lane L < 64: xslot of
// pair 8 (L + 64 c) + 2 j + h, written as the lane's base and an offset (2 j + h < 8 keeps (8 L + 2 j + h) / 32 at L / 4)
__device__ __forceinline__ int xq(int lane, int q, int h) { return 8 * lane + (lane >> 2) + 528 * (q >> 2) + 2 * (q & 3) + h; }

// Loads per lane in one polling round: at most 16 (64 registers of the control wave).
constexpr int mb(int n) { return n / 128 < 16 ? n / 128 : 16; }
// The activation's poll holds up to 24 loads per round (96 of the control wave's 256 registers): the 3072-cell
// activation of the hidden-1024 shape in one round (a second round trip costs about 0.5 us per exchange).
constexpr int mbh(int n) { return n / 128 < 24 ? n / 128 : 24; }

// ---- control wave: poll cells into LDS ---------------------------------------------------------------------
// Waits until cells [idx0, idx0 + n) (idx0 and n multiples of 128) all carry epoch e, copying the values to dst.
// Returns false on timeout or when the global error word is set.
template <int MAXB, bool SW = false, bool LO = false, bool SINGLE = false>
__device__ bool poll_cells(const void* region, uint32_t slots, uint32_t idx0, int n, uint32_t e, float* dst, void* ws,
                           int lane, const Ctx& c, uint32_t code, int f, int l) {
  for (uint32_t spin = 0;; spin++) {
    bool ok = true;
    for (int base = 0; base < n; base += 128 * MAXB) {
      u32x4 q[MAXB];
#pragma unroll
      for (int b = 0; b < MAXB; b++) {
        if (base + 128 * b < n)  // n is a multiple of 128: the condition is wave-uniform
          q[b] = LO ? get2l<SINGLE>(region, slots, idx0 + (uint32_t)(base + 128 * b), lane)
                    : get2v<SINGLE>(region, slots, idx0 + (uint32_t)(base + 128 * b), lane);
      }
#pragma unroll
      for (int b = 0; b < MAXB; b++) {
        const int i = base + 128 * b + 2 * lane;
        if (i < n) {
          ok &= q[b].y == e && q[b].w == e;
          const int o = SW ? xsw(i) : i;  // i even: i + 1 lands at o + 1
          dst[o] = __uint_as_float(q[b].x);
          dst[o + 1] = __uint_as_float(q[b].z);
        }
      }
    }
    if (__all(ok)) return true;
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

// ---- control wave: a whole vector into registers -----------------------------------------------------------
// Waits until cells [idx0, idx0 + 128 NB) (idx0 a multiple of 128) all carry epoch e. Lane holds cells 2 lane + 128 b and 2 lane + 128 b + 1
// in q[b].x and q[b].z; nothing goes through LDS here, the caller uses the values from registers (reading them
// back from LDS would cost one LDS round trip per dependent read). Returns false on timeout or when the global
// error word is set.
template <int NB, bool LO = false, bool SINGLE = false>
__device__ bool poll_regs(const void* region, uint32_t slots, uint32_t idx0, uint32_t e, u32x4 (&q)[NB], void* ws,
                          int lane, const Ctx& c, uint32_t code, int f, int l) {
  for (uint32_t spin = 0;; spin++) {
#pragma unroll
    for (int b = 0; b < NB; b++)
      q[b] = LO ? get2l<SINGLE>(region, slots, idx0 + (uint32_t)(128 * b), lane)
                : get2v<SINGLE>(region, slots, idx0 + (uint32_t)(128 * b), lane);
    bool ok = true;
#pragma unroll
    for (int b = 0; b < NB; b++) ok &= q[b].y == e && q[b].w == e;
    if (__all(ok)) return true;
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
template <int NB>
__device__ __forceinline__ void cells_to_pairs(const u32x4 (&q)[NB], float2 (&v)[NB]) {
#pragma unroll
  for (int b = 0; b < NB; b++) v[b] = make_float2(__uint_as_float(q[b].x), __uint_as_float(q[b].z));
}
// RMSNorm input staging from registers (lane holds elements 2 lane + 128 b and 2 lane + 128 b + 1 of the residual
// in v[b], and the norm weights of the same elements in w[b]): the residual to res (natural order, read back by the
// residual adds), the residual times the weights to xs (swizzled GEMV input), and the sum of squares of the whole
// vector as the result (wave-uniform). Every LDS write is issued without waiting for another.
template <int NB>
__device__ __forceinline__ float stage_rms(const float2 (&v)[NB], const float2 (&w)[NB], float* res, float* xs, int lane) {
  float ss = 0.f;
#pragma unroll
  for (int b = 0; b < NB; b++) {
    const int i = 2 * lane + 128 * b;  // even: its pair stays adjacent under the swizzle (xsw(i + 1) == xsw(i) + 1)
    *(float2*)(res + i) = v[b];
    *(float2*)(xs + xsw(i)) = make_float2(v[b].x * w[b].x, v[b].y * w[b].y);
    ss += v[b].x * v[b].x;
    ss += v[b].y * v[b].y;
  }
  return wave_sum(ss);
}
// A plain GEMV input from registers (lane holds elements 2 lane + 128 b, + 1 in v[b]) to xs, swizzled (xsw).
template <int NB>
__device__ __forceinline__ void stage_plain(const float2 (&v)[NB], float* xs, int lane) {
#pragma unroll
  for (int b = 0; b < NB; b++) *(float2*)(xs + xsw(2 * lane + 128 * b)) = v[b];
}
template <int NB>
__device__ __forceinline__ void load_pairs(const float* p, float2 (&w)[NB], int lane) {
#pragma unroll
  for (int b = 0; b < NB; b++) {
    const uint64_t u = gload((const uint64_t*)p + lane + 64 * b);  // elements 2 lane + 128 b, + 1
    w[b] = make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
  }
}

// ---- compute-wave GEMV pieces ------------------------------------------------------------------------------
// A wave owns RW consecutive rows starting at row0 (wave-uniform); lane reads chunk lane + 64 c of each row.
// The row scales come with the weights through vector loads (a scalar load would make every later LDS wait,
// lgkmcnt, wait for it as well) and stay raw bf16 bits until the dot that uses them: converting on arrival would
// make the wave wait for the load right after issuing it.
// A weight chunk through the caches (the code predictor's layers with keep_layers: read 16 times per frame).
__device__ __forceinline__ uint4 ld_keep(const uint4* p) {
  const u32x4 r = *(gptr<const u32x4>)p;
  return make_uint4(r.x, r.y, r.z, r.w);
}
template <int RW, int C, bool LO = false, bool KEEP = false>
__device__ __forceinline__ void load_rows(uint4 (&w)[RW][C], uint16_t (&s)[RW], const int8_t* W, const uint16_t* S,
                                          int row0, int nvalid, int K, int lane) {
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const int row = r < nvalid ? row0 + r : row0;
    if constexpr (LO) {  // row start in the scalar offset, lane bytes (+ chunk) in the shared vector offset
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)row * (uint32_t)K);
#pragma unroll
      for (int c = 0; c < C; c++)
        w[r][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(uniform(W)),
                                                                                  (uint32_t)lane * 16u + 1024u * c, so, KEEP ? 0 : kNT));
      s[r] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(uniform(S)), 0, __builtin_amdgcn_readfirstlane((uint32_t)row * 2u), 0);
      continue;
    }
    const uint4* p = (const uint4*)(W + (size_t)row * K);
#pragma unroll
    for (int c = 0; c < C; c++) w[r][c] = KEEP ? ld_keep(p + lane + 64 * c) : ld_stream(p + lane + 64 * c);
    // one ushort load per row: merged wider loads would be split into halves right away, waiting for them
    s[r] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(uniform(S)), (uint32_t)row * 2u, 0, 0);
  }
}
// y[r] = (row r) . xs, reduced over the wave (uniform result), without the row scale; xs is swizzled (xsw)
template <int RW, int C>
__device__ __forceinline__ void dot_rows(const uint4 (&w)[RW][C], const float* xs, int lane, float (&y)[RW]) {
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) acc[r] = 0.f;
  const float2* xs2 = (const float2*)xs;
#pragma unroll
  for (int c = 0; c < C; c++) {
#pragma unroll
    for (int j = 0; j < 4; j++) {  // one quarter of the chunk (4 bytes per row) at a time: 4 live x registers
      // two 8-byte LDS reads: 16-byte LDS reads stall the LDS on gfx950 (SQ_LDS_UNALIGNED_STALL; measured
      // 2250 against 820 cycles for the same 8 KB)
      const float2 u0 = xs2[xq(lane, 4 * c + j, 0)], u1 = xs2[xq(lane, 4 * c + j, 1)];
      const float4 v = make_float4(u0.x, u0.y, u1.x, u1.y);
#pragma unroll
      for (int r = 0; r < RW; r++) {
        const uint32_t q = j == 0 ? w[r][c].x : j == 1 ? w[r][c].y : j == 2 ? w[r][c].z : w[r][c].w;
        float t = (float)(int8_t)q * v.x;
        t = __builtin_fmaf((float)(int8_t)(q >> 8), v.y, t);
        t = __builtin_fmaf((float)(int8_t)(q >> 16), v.z, t);
        t = __builtin_fmaf((float)(int8_t)(q >> 24), v.w, t);
        acc[r] += t;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; r++) y[r] = wave_sum(acc[r]);
}

// Two GEMV inputs against the same rows (the code predictor's paired pass): each weight byte is converted once and
// multiplied with both inputs, as dot_rows does for one. The inputs are read one quarter chunk ahead of their use,
// with a scheduling barrier after each quarter: left free, the scheduler issues every LDS read of the dot first and
// holds all of them in registers (96 for the down rows), and the pass spills.
template <int RW, int C>
__device__ __forceinline__ void dot_rows2(const uint4 (&w)[RW][C], const float* xa, const float* xb, int lane,
                                          float (&ya)[RW], float (&yb)[RW]) {
  float aa[RW], ab[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) { aa[r] = 0.f; ab[r] = 0.f; }
  const float2* xa2 = (const float2*)xa;
  const float2* xb2 = (const float2*)xb;
  float2 na0 = xa2[xq(lane, 0, 0)], na1 = xa2[xq(lane, 0, 1)], nb0 = xb2[xq(lane, 0, 0)], nb1 = xb2[xq(lane, 0, 1)];
#pragma unroll
  for (int t = 0; t < 4 * C; t++) {  // quarter t: chunk t / 4, bytes 4 (t % 4) .. + 3 of each row's chunk
    const float2 a0 = na0, a1 = na1, b0 = nb0, b1 = nb1;
    if (t + 1 < 4 * C) {
      const int k0 = xq(lane, t + 1, 0), k1 = xq(lane, t + 1, 1);
      na0 = xa2[k0]; na1 = xa2[k1]; nb0 = xb2[k0]; nb1 = xb2[k1];
    }
    const int c = t >> 2, j = t & 3;
#pragma unroll
    for (int r = 0; r < RW; r++) {
      const uint32_t q = j == 0 ? w[r][c].x : j == 1 ? w[r][c].y : j == 2 ? w[r][c].z : w[r][c].w;
      const float w0 = (float)(int8_t)q, w1 = (float)(int8_t)(q >> 8), w2 = (float)(int8_t)(q >> 16),
                  w3 = (float)(int8_t)(q >> 24);
      float t0 = w0 * a0.x, u = w0 * b0.x;
      t0 = __builtin_fmaf(w1, a0.y, t0);
      u = __builtin_fmaf(w1, b0.y, u);
      t0 = __builtin_fmaf(w2, a1.x, t0);
      u = __builtin_fmaf(w2, b1.x, u);
      t0 = __builtin_fmaf(w3, a1.y, t0);
      u = __builtin_fmaf(w3, b1.y, u);
      aa[r] += t0;
      ab[r] += u;
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < RW; r++) { ya[r] = wave_sum(aa[r]); yb[r] = wave_sum(ab[r]); }
}

// i8g32 weights (the reference's format: one fp16 scale per 32 weights of a row, applied per 16-weight chunk,
// qwen3/kernels.py:104-110): a lane's chunk c of a row covers weights 16 (lane + 64 c) .. + 15, inside group
// (lane + 64 c) / 2, whose scale comes with the chunk (raw fp16 bits until the dot). KEEP as for load_rows.
template <int RW, int C, bool LO = false, bool KEEP = false>
__device__ __forceinline__ void load_rows_g32(uint4 (&w)[RW][C], uint16_t (&g)[RW][C], const int8_t* W, const uint16_t* S,
                                              int row0, int nvalid, int K, int lane) {
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const int row = r < nvalid ? row0 + r : row0;
    if constexpr (LO) {  // row starts in the scalar offsets; the scale of chunk c is at byte (lane & ~1) + 64 c
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)row * (uint32_t)K);
      const uint32_t sg = __builtin_amdgcn_readfirstlane((uint32_t)row * (uint32_t)(K >> 4));
#pragma unroll
      for (int c = 0; c < C; c++) {
        w[r][c] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(uniform(W)),
                                                                                  (uint32_t)lane * 16u + 1024u * c, so,
                                                                                  KEEP ? 0 : kNT));
        g[r][c] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(uniform(S)), ((uint32_t)lane & ~1u) + 64u * c, sg, 0);
      }
      continue;
    }
    const uint4* p = (const uint4*)(W + (size_t)row * K);
#pragma unroll
    for (int c = 0; c < C; c++) {
      w[r][c] = KEEP ? ld_keep(p + lane + 64 * c) : ld_stream(p + lane + 64 * c);
      g[r][c] = __builtin_amdgcn_raw_buffer_load_b16(make_rsrc(uniform(S)),
                                                     ((uint32_t)row * (uint32_t)(K >> 5) + (uint32_t)((lane + 64 * c) >> 1)) * 2u,
                                                     0, 0);
    }
  }
}
// y[r] = sum over the lane's chunks of (group scale) * (chunk . xs), reduced over the wave; xs swizzled (xsw)
template <int RW, int C>
__device__ __forceinline__ void dot_rows_g32(const uint4 (&w)[RW][C], const uint16_t (&g)[RW][C], const float* xs,
                                             int lane, float (&y)[RW]) {
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) acc[r] = 0.f;
  const float2* xs2 = (const float2*)xs;
#pragma unroll
  for (int c = 0; c < C; c++) {
    float part[RW];
#pragma unroll
    for (int r = 0; r < RW; r++) part[r] = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float2 u0 = xs2[xq(lane, 4 * c + j, 0)], u1 = xs2[xq(lane, 4 * c + j, 1)];
      const float4 v = make_float4(u0.x, u0.y, u1.x, u1.y);
#pragma unroll
      for (int r = 0; r < RW; r++) {
        const uint32_t q = j == 0 ? w[r][c].x : j == 1 ? w[r][c].y : j == 2 ? w[r][c].z : w[r][c].w;
        float t = (float)(int8_t)q * v.x;
        t = __builtin_fmaf((float)(int8_t)(q >> 8), v.y, t);
        t = __builtin_fmaf((float)(int8_t)(q >> 16), v.z, t);
        t = __builtin_fmaf((float)(int8_t)(q >> 24), v.w, t);
        part[r] += t;
      }
    }
#pragma unroll
    for (int r = 0; r < RW; r++) acc[r] = __builtin_fmaf(h2f(g[r][c]), part[r], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < RW; r++) y[r] = wave_sum(acc[r]);
}
// bf16 weights (the reference's Qwen3Kernels default, qwen3/kernels.py:434-437; no scales): a lane's chunk c of a
// row is still weights 16 (lane + 64 c) .. + 15, the same GEMV input layout as int8, held in two 16-byte loads
// (w[r][2c], w[r][2c + 1]). KEEP as for load_rows.
template <int RW, int C2, bool LO = false, bool KEEP = false>
__device__ __forceinline__ void load_rows_bf16(uint4 (&w)[RW][C2], const void* W, int row0, int nvalid, int K, int lane) {
  static_assert(C2 % 2 == 0, "two loads per chunk");
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const int row = r < nvalid ? row0 + r : row0;
    if constexpr (LO) {  // row start in the scalar offset, lane bytes (+ chunk) in the shared vector offset
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)row * (uint32_t)K * 2u);
#pragma unroll
      for (int c = 0; c < C2 / 2; c++)
#pragma unroll
        for (int h = 0; h < 2; h++)
          w[r][2 * c + h] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          make_rsrc(uniform(W)), (uint32_t)lane * 32u + 2048u * c + 16u * h,
                                                          so, KEEP ? 0 : kNT));
      continue;
    }
    const uint4* p = (const uint4*)((const char*)W + (size_t)row * K * 2);
#pragma unroll
    for (int c = 0; c < C2 / 2; c++)
#pragma unroll
      for (int h = 0; h < 2; h++)
        w[r][2 * c + h] = KEEP ? ld_keep(p + 2 * (lane + 64 * c) + h) : ld_stream(p + 2 * (lane + 64 * c) + h);
  }
}
__device__ __forceinline__ float bf_lo(uint32_t u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf_hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
// y[r] = (row r) . xs for bf16 rows, reduced over the wave; xs swizzled (xsw) as for int8
template <int RW, int C2>
__device__ __forceinline__ void dot_rows_bf16(const uint4 (&w)[RW][C2], const float* xs, int lane, float (&y)[RW]) {
  float acc[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) acc[r] = 0.f;
  const float2* xs2 = (const float2*)xs;
#pragma unroll
  for (int c = 0; c < C2 / 2; c++) {
#pragma unroll
    for (int j = 0; j < 4; j++) {  // weights 4 j .. 4 j + 3 of the chunk
      const float2 u0 = xs2[xq(lane, 4 * c + j, 0)], u1 = xs2[xq(lane, 4 * c + j, 1)];
#pragma unroll
      for (int r = 0; r < RW; r++) {
        const uint4 hq = w[r][2 * c + (j >> 1)];
        const uint32_t q0 = (j & 1) ? hq.z : hq.x, q1 = (j & 1) ? hq.w : hq.y;
        float t = bf_lo(q0) * u0.x;
        t = __builtin_fmaf(bf_hi(q0), u0.y, t);
        t = __builtin_fmaf(bf_lo(q1), u1.x, t);
        t = __builtin_fmaf(bf_hi(q1), u1.y, t);
        acc[r] += t;
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RW; r++) y[r] = wave_sum(acc[r]);
}
// dot_rows2 for bf16 rows (the code predictor's paired pass)
template <int RW, int C2>
__device__ __forceinline__ void dot_rows2_bf16(const uint4 (&w)[RW][C2], const float* xa, const float* xb, int lane,
                                               float (&ya)[RW], float (&yb)[RW]) {
  float aa[RW], ab[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) { aa[r] = 0.f; ab[r] = 0.f; }
  const float2* xa2 = (const float2*)xa;
  const float2* xb2 = (const float2*)xb;
  constexpr int Q = 4 * (C2 / 2);  // quarter chunks
  float2 na0 = xa2[xq(lane, 0, 0)], na1 = xa2[xq(lane, 0, 1)], nb0 = xb2[xq(lane, 0, 0)], nb1 = xb2[xq(lane, 0, 1)];
#pragma unroll
  for (int t = 0; t < Q; t++) {
    const float2 a0 = na0, a1 = na1, b0 = nb0, b1 = nb1;
    if (t + 1 < Q) {
      const int k0 = xq(lane, t + 1, 0), k1 = xq(lane, t + 1, 1);
      na0 = xa2[k0]; na1 = xa2[k1]; nb0 = xb2[k0]; nb1 = xb2[k1];
    }
    const int c = t >> 2, j = t & 3;
#pragma unroll
    for (int r = 0; r < RW; r++) {
      const uint4 hq = w[r][2 * c + (j >> 1)];
      const uint32_t q0 = (j & 1) ? hq.z : hq.x, q1 = (j & 1) ? hq.w : hq.y;
      const float w0 = bf_lo(q0), w1 = bf_hi(q0), w2 = bf_lo(q1), w3 = bf_hi(q1);
      float t0 = w0 * a0.x, u = w0 * b0.x;
      t0 = __builtin_fmaf(w1, a0.y, t0);
      u = __builtin_fmaf(w1, b0.y, u);
      t0 = __builtin_fmaf(w2, a1.x, t0);
      u = __builtin_fmaf(w2, b1.x, u);
      t0 = __builtin_fmaf(w3, a1.y, t0);
      u = __builtin_fmaf(w3, b1.y, u);
      aa[r] += t0;
      ab[r] += u;
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < RW; r++) { ya[r] = wave_sum(aa[r]); yb[r] = wave_sum(ab[r]); }
}
// Weight-format dispatch of the compute waves: i8row keeps one bf16 scale per row (applied by the caller through
// row_scale), i8g32 one fp16 scale per chunk (applied inside the dot; row_scale is then 1), bf16 none (row_scale 1,
// the chunk count C doubled by CfgW). The group-scale arrays of the i8row and bf16 kernels are [1][1] and unused.
template <int WD, int RW, int C, bool LO = false, bool KEEP = false, int GR, int GC>
__device__ __forceinline__ void load_w(uint4 (&w)[RW][C], uint16_t (&s)[RW], uint16_t (&g)[GR][GC], const int8_t* W,
                                       const uint16_t* S, int row0, int nvalid, int K, int lane) {
  if constexpr (WD == SK_WD_BF16) load_rows_bf16<RW, C, LO, KEEP>(w, W, row0, nvalid, K, lane);
  else if constexpr (WD == SK_WD_I8G32) load_rows_g32<RW, C, LO, KEEP>(w, g, W, S, row0, nvalid, K, lane);
  else load_rows<RW, C, LO, KEEP>(w, s, W, S, row0, nvalid, K, lane);
}
template <int WD, int RW, int C, int GR, int GC>
__device__ __forceinline__ void dot_w(const uint4 (&w)[RW][C], const uint16_t (&g)[GR][GC], const float* xs, int lane,
                                      float (&y)[RW]) {
  if constexpr (WD == SK_WD_BF16) dot_rows_bf16<RW, C>(w, xs, lane, y);
  else if constexpr (WD == SK_WD_I8G32) dot_rows_g32<RW, C>(w, g, xs, lane, y);
  else dot_rows<RW, C>(w, xs, lane, y);
}
// dot_rows2 for i8g32 weights: each chunk's sums of both inputs are scaled by the chunk's group scale, as
// dot_rows_g32 does for one input.
template <int RW, int C>
__device__ __forceinline__ void dot_rows2_g32(const uint4 (&w)[RW][C], const uint16_t (&g)[RW][C], const float* xa,
                                              const float* xb, int lane, float (&ya)[RW], float (&yb)[RW]) {
  float aa[RW], ab[RW], pa[RW], pb[RW];
#pragma unroll
  for (int r = 0; r < RW; r++) { aa[r] = 0.f; ab[r] = 0.f; pa[r] = 0.f; pb[r] = 0.f; }
  const float2* xa2 = (const float2*)xa;
  const float2* xb2 = (const float2*)xb;
  float2 na0 = xa2[xq(lane, 0, 0)], na1 = xa2[xq(lane, 0, 1)], nb0 = xb2[xq(lane, 0, 0)], nb1 = xb2[xq(lane, 0, 1)];
#pragma unroll
  for (int t = 0; t < 4 * C; t++) {  // quarter t: chunk t / 4, bytes 4 (t % 4) .. + 3 of each row's chunk
    const float2 a0 = na0, a1 = na1, b0 = nb0, b1 = nb1;
    if (t + 1 < 4 * C) {
      const int k0 = xq(lane, t + 1, 0), k1 = xq(lane, t + 1, 1);
      na0 = xa2[k0]; na1 = xa2[k1]; nb0 = xb2[k0]; nb1 = xb2[k1];
    }
    const int c = t >> 2, j = t & 3;
#pragma unroll
    for (int r = 0; r < RW; r++) {
      const uint32_t q = j == 0 ? w[r][c].x : j == 1 ? w[r][c].y : j == 2 ? w[r][c].z : w[r][c].w;
      const float w0 = (float)(int8_t)q, w1 = (float)(int8_t)(q >> 8), w2 = (float)(int8_t)(q >> 16),
                  w3 = (float)(int8_t)(q >> 24);
      float t0 = w0 * a0.x, u = w0 * b0.x;
      t0 = __builtin_fmaf(w1, a0.y, t0);
      u = __builtin_fmaf(w1, b0.y, u);
      t0 = __builtin_fmaf(w2, a1.x, t0);
      u = __builtin_fmaf(w2, b1.x, u);
      t0 = __builtin_fmaf(w3, a1.y, t0);
      u = __builtin_fmaf(w3, b1.y, u);
      pa[r] += t0;
      pb[r] += u;
      if (j == 3) {
        const float sc = h2f(g[r][c]);
        aa[r] = __builtin_fmaf(sc, pa[r], aa[r]);
        ab[r] = __builtin_fmaf(sc, pb[r], ab[r]);
        pa[r] = 0.f;
        pb[r] = 0.f;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int r = 0; r < RW; r++) { ya[r] = wave_sum(aa[r]); yb[r] = wave_sum(ab[r]); }
}
template <int WD, int RW, int C, int GR, int GC>
__device__ __forceinline__ void dot2_w(const uint4 (&w)[RW][C], const uint16_t (&g)[GR][GC], const float* xa,
                                       const float* xb, int lane, float (&ya)[RW], float (&yb)[RW]) {
  if constexpr (WD == SK_WD_BF16) dot_rows2_bf16<RW, C>(w, xa, xb, lane, ya, yb);
  else if constexpr (WD == SK_WD_I8G32) dot_rows2_g32<RW, C>(w, g, xa, xb, lane, ya, yb);
  else dot_rows2<RW, C>(w, xa, xb, lane, ya, yb);
}
template <int WD>
__device__ __forceinline__ float row_scale_of(uint16_t s) {
  if constexpr (WD == SK_WD_I8G32 || WD == SK_WD_BF16) return 1.f;
  else return bf2f(s);
}

// Publishes a stage's outputs. Every compute wave has left its values in S.pub (lane 0, before the call); the last
// wave to arrive writes the workgroup's n cells [idx0, idx0 + n) (idx0 and n even, n <= 64) with 16-byte stores,
// so each line of cells is written by one wave at one time (lines written piecewise by several waves reach the
// pollers later). ALL: cells every XCD reads, stored into all eight pages of their period, lane k storing pair
// j0 + k / 8 into page k % 8 (one store instruction per 8 pairs; eight stores per lane, or pages by lane with a
// division by the pair count, made the kernels spill more and run slower), or with SINGLE into their one copy;
// otherwise this XCD's copy. There is no barrier: the control wave may be polling the next stage's input meanwhile.
template <int W, bool ALL, bool SINGLE = false, class L>
__device__ __forceinline__ void publish(L& S, void* region, uint32_t slots, uint32_t idx0, int n, uint32_t e, int lane) {
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(&S.pubcnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old % W == W - 1) {
    const int pieces = n / 2;
    if constexpr (ALL && !SINGLE) {
#pragma unroll
      for (int j0 = 0; j0 < 32; j0 += 8) {  // lane: page lane % 8 of pair j0 + lane / 8
        const int j = j0 + (lane >> 3);
        if (j0 < pieces && j < pieces) {
          const u32x4 v = {__float_as_uint(S.pub[2 * j]), e, __float_as_uint(S.pub[2 * j + 1]), e};
          __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(region),
                                                 ((uint32_t)(lane & 7) << 12) + cell_off(idx0 + 2u * (uint32_t)j), 0, kPolDev);
        }
      }
    } else if (lane < pieces) {
      const u32x4 v = {__float_as_uint(S.pub[2 * lane]), e, __float_as_uint(S.pub[2 * lane + 1]), e};
      const uint32_t i = idx0 + 2u * (uint32_t)lane;
      __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(region), ALL ? single_off(i) : own_off(slots, i), 0, kPolDev);
    }
    if (lane == 0) __hip_atomic_store(&S.pubseq, (old + 1) / W, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// publish for the paired pass (the hidden-1024 code predictor): S.pub holds the first row's n values, then the second
// row's; the last wave to arrive writes them to cells [idxA, idxA + n) and [idxB, idxB + n) (ALL as for publish, the
// pages by lane). One publication (one pubseq step) for both rows.
template <int W, bool ALL, class L>
__device__ __forceinline__ void publish_pair(L& S, void* region, uint32_t slots, uint32_t idxA, uint32_t idxB, int n,
                                             uint32_t e, int lane) {
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(&S.pubcnt, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old % W == W - 1) {
    const int pieces = n / 2, per_row = (ALL ? 8 : 1) * pieces;
    for (int k = lane; k < 2 * per_row; k += 64) {
      const int row = k >= per_row ? 1 : 0, kr = k - row * per_row;
      const int pg = kr / pieces, j = kr - pg * pieces;
      const u32x4 v = {__float_as_uint(S.pub[row * n + 2 * j]), e, __float_as_uint(S.pub[row * n + 2 * j + 1]), e};
      const uint32_t i = (row ? idxB : idxA) + 2u * (uint32_t)j;
      __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(region), ALL ? ((uint32_t)pg << 12) + cell_off(i) : own_off(slots, i),
                                             0, kPolDev);
    }
    if (lane == 0) __hip_atomic_store(&S.pubseq, (old + 1) / W, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

// Sleeps n units of 64 shader clocks.
__device__ __forceinline__ void sleep_units(uint32_t n) {
  for (uint32_t i = 0; i < n; i++) __builtin_amdgcn_s_sleep(1);
}
// Control wave: waits in LDS (no memory traffic) until this workgroup's compute waves have completed `seq` stage
// publications, then `delay` sleep units more. Bounded: a wait that outlasts ~30 ms falls through and the poll
// that follows reports the error.
template <class L>
__device__ __forceinline__ void after_publish(L& S, uint32_t seq, uint32_t delay) {
  for (uint32_t i = 0; i < (1u << 20); i++) {
    if (__hip_atomic_load(&S.pubseq, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= seq) break;
    __builtin_amdgcn_s_sleep(1);
  }
  sleep_units(delay);
}

// ---- control wave: sampled pick ---------------------------------------------------------------------------
// Integer wave64 reductions over DPP (every lane's value; the results are wave-uniform).
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ uint32_t dppu(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  v += dppu<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dppu<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dppu<0x124>(v);  // row_ror:4
  v += dppu<0x128>(v);  // row_ror:8
  v += dppu<0x142, 0xA>(v);  // row_bcast:15
  v += dppu<0x143, 0xC>(v);  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dppu<0xB1>(v));
  v = max(v, dppu<0x4E>(v));
  v = max(v, dppu<0x124>(v));
  v = max(v, dppu<0x128>(v));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)v, 0), b = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)v, 32), d = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
// Inclusive prefix sum over the 64 lanes (row_shr within rows of 16, then row_bcast across rows).
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  // Hillis-Steele within each row of 16 (a source lane outside the row reads as 0), then the row totals carried
  // across rows: lane 15 of rows 0 / 2 into rows 1 / 3, then lane 31 (rows 0-1) into rows 2 and 3
  v += dppu<0x111>(v);        // row_shr:1
  v += dppu<0x112>(v);        // row_shr:2
  v += dppu<0x114>(v);        // row_shr:4
  v += dppu<0x118>(v);        // row_shr:8
  v += dppu<0x142, 0xA>(v);  // row_bcast:15
  v += dppu<0x143, 0xC>(v);  // row_bcast:31
  return v;
}

// The largest key t in [lo, hi] whose count c(t) (keys >= t) reaches K, given c(lo) >= K and c(hi + 1) < K. Bits
// above the highest bit where lo and hi differ are common to every such t; below it the prefix grows one bit at a
// time, the bit kept when the count at the prefix with the bit set reaches K.
template <class F>
__device__ __forceinline__ uint32_t bisect_keys(uint32_t lo, uint32_t hi, uint32_t K, F count) {
  if (lo >= hi) return lo;
  const int top = 31 - __builtin_clz(lo ^ hi);
  uint32_t p = top == 31 ? 0u : lo & ~((2u << top) - 1u);
  for (int b = top; b >= 0; b--) {
    const uint32_t t = p | (1u << b);
    if (count(t) >= K) p = t;
  }
  return p;
}

// LDS that a sampled pick's control wave and compute waves share, after the LDS copy of the value cells (sampling
// instantiations only).
struct PickShared {
  uint32_t lm[64];  // the control wave's 64 lane maxima, for the bound's ranks
  uint32_t lb;      // lower bound of the threshold key
  uint32_t n;       // candidates compacted (LDS atomic; zeroed by the control wave before the compaction)
  uint32_t bad;     // nonzero: a poll failed and there is no pick (zeroed at launch and after each pick)
  uint32_t pad;
  float gv[4];      // per compute wave: the largest perturbed value among its kept candidates (-inf: none)
  uint32_t bi[4];   // the lowest index holding it (0x7fffffff: none)
  uint32_t nk[4];   // kept candidates per compute wave
};
static_assert(offsetof(PickShared, gv) % 16 == 0 && offsetof(PickShared, bi) == offsetof(PickShared, gv) + 16 &&
                  offsetof(PickShared, nk) == offsetof(PickShared, gv) + 32,
              "the combine reads gv, bi and nk as three 16-byte vectors");
template <int H, int I, int W, int V, bool CP>
constexpr size_t kPickShared = kPickCopy<H, I, W, V, CP> + (size_t)V * 8;
constexpr uint32_t kNegInfKey = 0x007fffffu;  // order_key(-inf)
// The value whose order key is k (order_key is a bijection).
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? k ^ 0x80000000u : ~k);
}
typedef __attribute__((address_space(3))) float lds_f32;
typedef __attribute__((address_space(3))) uint16_t lds_u16;
typedef __attribute__((address_space(3))) uint32_t lds_u32;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) PickShared lds_pick;
// The LDS address of p (a pointer into the workgroup's LDS) as a value the compiler cannot trace back to the
// kernel's dynamic LDS array: an out-of-line function handed an address derived from that array looks the array's
// base up in a per-kernel table in memory, again after every LDS store it cannot rule out as aliasing.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  uint32_t a = (uint32_t)(size_t)(const __attribute__((address_space(3))) char*)p;
  __asm__ volatile("" : "+s"(a));
  return a;
}
template <class T>
__device__ __forceinline__ T* lds_at(uint32_t a) {  // an LDS pointer from an lds_addr value
  return (T*)(size_t)__builtin_amdgcn_readfirstlane(a);
}

// A sampled pick draws as the fused sampler does: the key of the top_k-th largest of the V processed logits (ties
// kept; top_k <= 0 or >= V keeps everything), then the largest v - log(-log u) over the kept values that are not
// -inf, u from Philox draw `draw` under key `seed`, lowest index on ties, 0 if nothing is kept. Every workgroup
// publishes its ROWS values (cells vals + ROWS g ..) and their largest order key (cell maxs + g), and every
// workgroup computes the same pick from all of them, the control wave and the compute waves together:
//
//  1. control wave: publish, poll the 256 maxima (lane l holds workgroups 2l, 2l+1, 128+2l, 129+2l) and, for
//     top_k <= 64, take the top_k-th largest of the 64 lane maxima as a lower bound lb of the threshold (they are
//     64 of the values): the largest lane maximum that at least top_k lane maxima reach, one rank per lane.
//     Compute waves, meanwhile: each loads a quarter of the V value cells straight into LDS (cb, a copy of the
//     cells; direct loads hold no registers) and re-loads it until every epoch is the frame's.
//  2. compute waves: the indices and keys of their values >= lb are appended to ci / ck (a scan over the lanes,
//     one LDS atomic per wave for the wave's place; the order does not matter below).
//  3. compute waves, when 0 < top_k <= 64 and at most 256 candidates: candidate j (lane j % 64 of wave j / 64) is
//     kept iff fewer than top_k candidates have a larger key (every key above lb is a candidate, so this is the
//     rank among all V values, and key >= threshold); kept candidates draw their Philox noise and each wave
//     reduces its largest perturbed value and lowest index. The control wave combines the four.
//     Otherwise the control wave finds the threshold by bisection of the keys over the candidates (ballot
//     counts), compacts the kept ones and draws alone (keep-all, top_k > 64, or a bound that leaves more than
//     256 candidates, as when many values tie).
// Three workgroup barriers separate the steps; both roles pass all three whatever happens, and a failed poll
// only sets `bad`. A single wave pays about 90 cycles for each comparison that feeds a ballot and issues one
// instruction every few cycles, so the steps that scale with the candidates run on the four compute waves
// (4 x 64 lanes) and the control wave keeps the parts that do not.

// Control wave. Kept out of line (one call per frame) and only in the sampling instantiation of the kernel. The
// arguments arrive in vector registers under the call convention; they are made wave-uniform first so the control
// flow stays scalar. Returns the pick, -1 when the error word is set or a compute wave's poll failed, -2 when the
// maxima poll timed out. `tp` (null unless tracing) receives wall-clock stamps (tp[10..14]) and shader-clock stamps
// (tp[0..4]) after the bound, the compaction, the ranks and draws, the fallback's kept compaction and the pick, and
// lb and the counts of candidates and kept values (tp[5..7]).
template <int V, int ROWS, bool SINGLE = false>
__device__ __attribute__((noinline)) int64_t sampled_pick(char* region_, uint32_t slots_, uint32_t vals_,
                                                          uint32_t maxs_, int g_, uint32_t e_, uint32_t hv_,
                                                          uint32_t cb_, uint32_t ci_, uint32_t ck_, uint32_t ps_,
                                                          int top_k_, uint64_t draw_, uint64_t seed_, void* ws_,
                                                          uint32_t delay_, int lane, uint64_t* tp_) {
  static_assert(V % 512 == 0 && V == ROWS * kWG && ROWS % 2 == 0 && ROWS <= 16, "vocabulary of 256 x ROWS");
  char* region = uniform(region_);
  const uint32_t slots = __builtin_amdgcn_readfirstlane(slots_);
  void* ws = uniform(ws_);
  gptr<uint64_t> tp = (gptr<uint64_t>)uniform(tp_);
  const lds_f32* hv = lds_at<const lds_f32>(hv_);
  const lds_f32* cbf = lds_at<const lds_f32>(cb_);  // LDS arrays: ds_* accesses rather than flat
  auto cv = [&](uint32_t i) { return cbf[2 * i]; };  // value i: word 0 of its cell's LDS copy
  lds_u16* ci = lds_at<lds_u16>(ci_);                // candidate indices [V]
  const lds_u32* ck = lds_at<const lds_u32>(ck_);    // their keys [V]
  lds_pick* ps = lds_at<lds_pick>(ps_);
  const uint32_t maxs = __builtin_amdgcn_readfirstlane(maxs_);
  const uint32_t vals = __builtin_amdgcn_readfirstlane(vals_);
  const uint32_t e = __builtin_amdgcn_readfirstlane(e_);
  const int g = __builtin_amdgcn_readfirstlane(g_);
  const int top_k = __builtin_amdgcn_readfirstlane(top_k_);
  const uint32_t delay = __builtin_amdgcn_readfirstlane(delay_);
  const uint32_t d0 = __builtin_amdgcn_readfirstlane((uint32_t)draw_), d1 = __builtin_amdgcn_readfirstlane((uint32_t)(draw_ >> 32));
  const uint32_t k0 = __builtin_amdgcn_readfirstlane((uint32_t)seed_), k1 = __builtin_amdgcn_readfirstlane((uint32_t)(seed_ >> 32));
  const uint64_t draw = ((uint64_t)d1 << 32) | d0;
  const bool keep_all = top_k <= 0 || top_k >= V;
  const uint32_t K = (uint32_t)top_k;

  // (1) publish the values, then this workgroup's largest key; poll the maxima; the bound
  const float own = lane < ROWS ? hv[lane] : -INFINITY;
  const uint32_t own_max = wave_max_u32(lane < ROWS ? order_key(own) : 0u);
  // the values into all eight pages: lane k < 4 ROWS stores pair k % (ROWS / 2) into page k / (ROWS / 2); the
  // maximum: lane k < 8 into page k (SINGLE: the one copy, lanes k < ROWS / 2 and lane 0)
  constexpr int kPages = SINGLE ? 1 : 8;
  if (lane < kPages * (ROWS / 2)) {
    const int pg = lane / (ROWS / 2), j = lane - pg * (ROWS / 2);
    const u32x4 v = {__float_as_uint(hv[2 * j]), e, __float_as_uint(hv[2 * j + 1]), e};
    const uint32_t i = vals + (uint32_t)(ROWS * g + 2 * j);
    __builtin_amdgcn_raw_buffer_store_b128(v, make_rsrc(region), SINGLE ? single_off(i) : ((uint32_t)pg << 12) + cell_off(i), 0,
                                           kPolDev);
  }
  if (lane < kPages) {
    const u32x2 v = {own_max, e};
    const uint32_t i = maxs + (uint32_t)g;
    __builtin_amdgcn_raw_buffer_store_b64(v, make_rsrc(region), SINGLE ? single_off(i) : ((uint32_t)lane << 12) + cell_off(i), 0,
                                          kPolDev);
  }
  if (lane == 0) ps->n = 0u;
  sleep_units(delay);
  int rc = 0;
  u32x4 mq[2];
  for (uint32_t spin = 0;; spin++) {
    mq[0] = get2<SINGLE>(region, slots, maxs + (uint32_t)(2 * lane));
    mq[1] = get2<SINGLE>(region, slots, maxs + (uint32_t)(128 + 2 * lane));
    if (__all(mq[0].y == e && mq[0].w == e && mq[1].y == e && mq[1].w == e)) break;
    if ((spin & 63) == 63) {
      if (ld_u32_dev(ws, Ws::kErr) != 0) { rc = -1; break; }
      if (spin > kSpinLimit) { rc = -2; break; }
    }
    __builtin_amdgcn_s_sleep(1);
  }
  const uint32_t lm = max(max(mq[0].x, mq[0].z), max(mq[1].x, mq[1].z));  // the maxima are order keys already
  const uint32_t top_key = wave_max_u32(lm);                               // the largest key of all
  uint32_t lb = 0;
  if (rc == 0 && !keep_all && top_k <= 64) {
    ps->lm[lane] = lm;
    const lds_u32x4* lm4 = (const lds_u32x4*)ps->lm;
    uint32_t ge = 0;  // lane maxima >= this lane's
#pragma unroll
    for (int q = 0; q < 16; q++) {
      const u32x4 m4 = lm4[q];
      ge += (uint32_t)(m4.x >= lm) + (uint32_t)(m4.y >= lm) + (uint32_t)(m4.z >= lm) + (uint32_t)(m4.w >= lm);
    }
    lb = wave_max_u32(ge >= K ? lm : 0u);  // the top_k-th largest lane maximum
  }
  if (lane == 0) {
    ps->lb = lb;
    if (rc != 0) __hip_atomic_fetch_or(&ps->bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  // stamps are kept in registers and stored at the end: a global store in flight would hold up the next wait
  uint64_t st[16] = {};
  const bool trc = tp != nullptr;
  if (trc) { st[10] = (uint64_t)wall_clock64(); st[0] = (uint64_t)clock64(); }
  wg_sync();  // (1) done: the values are in LDS, lb is set
  wg_sync();  // (2) done: candidates compacted
  const uint32_t n = __builtin_amdgcn_readfirstlane(ps->n);
  const bool bad = __builtin_amdgcn_readfirstlane(ps->bad) != 0;
  const bool fast = !bad && !keep_all && top_k <= 64 && n <= 256u;
  if (trc) { st[11] = (uint64_t)wall_clock64(); st[1] = (uint64_t)clock64(); }
  wg_sync();  // (3) done: ranks and draws of the compute waves
  if (lane == 0) ps->bad = 0u;  // every wave has read it
  if (bad) return rc == -2 ? -2 : -1;
  if (trc) { st[12] = (uint64_t)wall_clock64(); st[2] = (uint64_t)clock64(); }
  uint32_t nk = 0;
  uint32_t pick;
  if (fast) {
    const lds_u32x4* r4 = (const lds_u32x4*)ps->gv;  // gv[4], bi[4], nk[4]: three 16-byte reads
    const u32x4 gq = r4[0], bq = r4[1], nq = r4[2];
    const float g0 = __uint_as_float(gq.x), g1 = __uint_as_float(gq.y), g2 = __uint_as_float(gq.z),
                g3 = __uint_as_float(gq.w);
    const float gmax = fmaxf(fmaxf(g0, g1), fmaxf(g2, g3));
    pick = min(min(g0 == gmax ? bq.x : 0x7fffffffu, g1 == gmax ? bq.y : 0x7fffffffu),
               min(g2 == gmax ? bq.z : 0x7fffffffu, g3 == gmax ? bq.w : 0x7fffffffu));
    pick = __builtin_amdgcn_readfirstlane(pick);
    nk = __builtin_amdgcn_readfirstlane((nq.x + nq.y) + (nq.z + nq.w));
    if (trc) { st[13] = st[12]; st[3] = st[2]; }
  } else {
    // the threshold: a bisection of the keys over the candidates (counts are ballots of one comparison each, with
    // the number of comparisons per step fixed outside the bisection: a branch per step costs more than a ballot)
    const int nm = (int)((n + 63) / 64);
    uint32_t thr = 0;
    if (!keep_all) {
      constexpr int kReg = 4;  // candidate keys held in registers; the rest are read from LDS
      uint32_t kk[kReg];
#pragma unroll
      for (int m = 0; m < kReg; m++) {
        const uint32_t j = (uint32_t)(lane + 64 * m);
        kk[m] = j < n ? ck[j] : 0u;  // 0 never counts: every probed key t is at least 1
      }
      if (nm <= 4) {
        thr = bisect_keys(lb, top_key, K, [&](uint32_t t) {
          return (uint32_t)__popcll(__ballot(kk[0] >= t)) + (uint32_t)__popcll(__ballot(kk[1] >= t)) +
                 (uint32_t)__popcll(__ballot(kk[2] >= t)) + (uint32_t)__popcll(__ballot(kk[3] >= t));
        });
      } else {
        thr = bisect_keys(lb, top_key, K, [&](uint32_t t) {
          uint32_t c = 0;
#pragma unroll
          for (int m = 0; m < kReg; m++) c += (uint32_t)__popcll(__ballot(kk[m] >= t));
          for (int m = kReg; m < nm; m++) {
            const uint32_t j = (uint32_t)(lane + 64 * m);
            c += (uint32_t)__popcll(__ballot(j < n && ck[j] >= t));
          }
          return c;
        });
      }
    }
    // the kept candidates (key >= thr, not -inf), compacted in place: a batch writes below its own start or over
    // itself, after all its lanes have read their entries
    for (int m = 0; m < nm; m++) {
      const uint32_t j = (uint32_t)(lane + 64 * m);
      uint32_t i = 0;
      bool take = false;
      if (j < n) {
        i = ci[j];
        const float x = cv(i);
        take = order_key(x) >= thr && x != -INFINITY;
      }
      const uint64_t msk = __ballot(take);
      if (take) ci[nk + __builtin_amdgcn_mbcnt_hi((uint32_t)(msk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)msk, 0u))] = (uint16_t)i;
      nk += (uint32_t)__popcll(msk);
    }
    if (trc) { st[13] = (uint64_t)wall_clock64(); st[3] = (uint64_t)clock64(); }
    // Gumbel-max: the largest perturbed value, then the lowest index among the lanes that hold it
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (uint32_t j = (uint32_t)lane; j < nk; j += 64) {
      const int i = (int)ci[j];
      const float gv = gumbel(cv(i), (uint32_t)i, draw, k0, k1);
      if (gv > best || (gv == best && i < bi)) { best = gv; bi = i; }
    }
    const float gmax = wave_max(best);
    pick = ~wave_max_u32(best == gmax ? ~(uint32_t)bi : 0u);
  }
  if (trc) {
    st[14] = (uint64_t)wall_clock64();
    st[4] = (uint64_t)clock64();
    st[5] = lb;
    st[6] = n;
    st[7] = nk;
    if (lane == 0) {
#pragma unroll
      for (int k = 0; k < 15; k++)
        if (k != 8 && k != 9) tp[k] = st[k];
    }
  }
  return pick == 0x7fffffffu || nk == 0 ? 0 : (int64_t)pick;
}

// Position bookkeeping of a frame for this workgroup's attention chunk.
// Positions [t0, t0 + n) of the cache (T = pos + 1 positions) that workgroup r of a head attends over: the cache
// split 32 ways; the owner of `pos` appends its K/V row.
struct Chunk {
  static constexpr bool whole = false;
  int T, pos, t0, n;
  __device__ Chunk(int pos_, int r) {
    pos = pos_;
    T = pos + 1;
    const int ch = (T + kChunks - 1) / kChunks;
    t0 = r * ch;
    const int t1 = min(T, t0 + ch);
    n = t1 > t0 ? t1 - t0 : 0;
  }
  __device__ bool has_pos() const { return n > 0 && t0 <= pos && pos < t0 + n; }
};
// The code predictor's chunk: when `whole` (a cache no longer than one workgroup's capacity) every workgroup of
// the head attends over the whole cache, so no partials are merged, and workgroup 0 of the head appends the row.
struct CpChunk {
  int T, pos, t0, n;
  bool whole, r0;
  __device__ CpChunk(int pos_, int r, bool whole_) {
    pos = pos_;
    T = pos + 1;
    const int ch = whole_ ? T : (T + kChunks - 1) / kChunks;
    t0 = whole_ ? 0 : r * ch;
    const int t1 = min(T, t0 + ch);
    n = t1 > t0 ? t1 - t0 : 0;
    whole = whole_;
    r0 = r == 0;
  }
  __device__ bool has_pos() const { return whole ? r0 : n > 0 && t0 <= pos && pos < t0 + n; }
};
template <bool CP>
using ChunkOf = typename std::conditional<CP, CpChunk, Chunk>::type;
template <bool CP>
__device__ __forceinline__ ChunkOf<CP> make_chunk(int pos, int r, bool whole) {
  if constexpr (CP) return CpChunk(pos, r, whole);
  else return Chunk(pos, r);
}

// Reduce-scatter of 16 values over the 16 lanes of a row: lane i of the row returns the row's sum of v[i]. Four
// exchanges between partner lanes (row_mirror i <-> 15 - i, row_half_mirror i <-> 7 - i within each half, then
// xor 2 and xor 1), each partner keeping the half of its values selected by the lane bit that tells it from the
// other (bits 3, 2, 1, 0 in turn) and adding the partner's copy of that half: 15 DPP adds instead of the 64 of 16
// row sums.
__device__ __forceinline__ float row16_reduce_scatter(const float (&v)[16], int lane) {
  float a[8], b[4], c[2];
  const bool h3 = lane & 8, h2 = lane & 4, h1 = lane & 2, h0 = lane & 1;
#pragma unroll
  for (int j = 0; j < 8; j++) a[j] = (h3 ? v[8 + j] : v[j]) + dpp<0x140>(h3 ? v[j] : v[8 + j]);  // row_mirror
#pragma unroll
  for (int j = 0; j < 4; j++) b[j] = (h2 ? a[4 + j] : a[j]) + dpp<0x141>(h2 ? a[j] : a[4 + j]);  // row_half_mirror
#pragma unroll
  for (int j = 0; j < 2; j++) c[j] = (h1 ? b[2 + j] : b[j]) + dpp<0x4E>(h1 ? b[j] : b[2 + j]);  // quad_perm [2,3,0,1]
  return (h0 ? c[1] : c[0]) + dpp<0xB1>(h0 ? c[0] : c[1]);  // quad_perm [1,0,3,2]
}

template <int W, int KVL, class Ck>
__device__ __forceinline__ void load_kv(uint4 (&kr)[KVL], uint4 (&vr)[KVL], const bf16_t* Kh, const bf16_t* Vh,
                                        const Ck& ck, int w, int g, int sl) {
// K by position: lane (g, sl) of wave w holds dims 8 sl .. + 7 of position t0 + 4 W i + 4 w + g. V goes by
// dimension slice: the same lane holds dims 32 w + 8 g .. + 7 of position t0 + sl + 16 i (each wave multiplies its
// 32 dims with every position's weight, so no partial sum crosses waves).
// Loads are unconditional, from a position clamped to ck.pos (< max_len): a load under a condition would need a
// select on its result, and a select makes the wave wait for the load at once. Slots beyond the chunk and the
// slot of `pos` itself (not written yet) are never read back: the attention code skips or replaces them.
#pragma unroll
  for (int i = 0; i < KVL; i++) {
    const int jj = 4 * W * i + 4 * w + g;
    const int t = min(ck.t0 + jj, ck.pos);
    const uint32_t off = (uint32_t)(t * SK_HD + 8 * sl) * 2u;
    kr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(uniform(Kh)), off, 0, kPolDev));
    const int tv = min(ck.t0 + sl + 16 * i, ck.pos);
    const uint32_t ov = (uint32_t)(tv * SK_HD + 32 * w + 8 * g) * 2u;
    vr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(uniform(Vh)), ov, 0, kPolDev));
  }
}

// K/V of a code-predictor launch of at most 16 positions (F16), for one workgroup's attention slice: lane
// 16 qq + j holds dims 32 qq .. 32 qq + 31 of K at position j (four 16-byte loads) and dims d0 + 2 qq, + 1 of V
// (one 4-byte load). Positions beyond npos load position npos (< max_len): unconditional loads, as load_kv.
__device__ __forceinline__ void load_kv16(uint4 (&kf)[4], uint32_t& vf, const bf16_t* Kh, const bf16_t* Vh, int npos,
                                          int d0, int lane) {
  const int j = lane & 15, qq = lane >> 4;
  const int t = min(j, npos);
  const uint32_t ko = (uint32_t)(t * SK_HD + 32 * qq) * 2u;
#pragma unroll
  for (int e = 0; e < 4; e++)
    kf[e] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(make_rsrc(uniform(Kh)), ko + 16u * e, 0, kPolDev));
  vf = __builtin_amdgcn_raw_buffer_load_b32(make_rsrc(uniform(Vh)), (uint32_t)(t * SK_HD + d0 + 2 * qq) * 2u, 0, kPolDev);
}

__device__ __forceinline__ void unpack8(uint4 a, float* o) {
  o[0] = bf2f(a.x & 0xffffu); o[1] = bf2f(a.x >> 16); o[2] = bf2f(a.y & 0xffffu); o[3] = bf2f(a.y >> 16);
  o[4] = bf2f(a.z & 0xffffu); o[5] = bf2f(a.z >> 16); o[6] = bf2f(a.w & 0xffffu); o[7] = bf2f(a.w >> 16);
}

// Code-predictor launch (CP): per-position inputs and heads. Position 0 takes the vector x0, position g >= 1
// the row of table emb[g] chosen by the previous code (code 0 for g = 1) and ends in head g; the codes go to
// d.out. Unused (all null) for the talker.
struct CpArgs {
  const float* x0;
  const void* const* emb;     // [n_positions] device array of bf16 tables; [0] unused
  const void* const* head_w;  // [n_positions] int8 heads; [0] unused
  const void* const* head_s;  // [n_positions] bf16 row scales
  int emb0_rows;              // rows of emb[1] (the range code 0 must lie in)
  int pair;                   // positions 0 and 1 in one pass (two rows per stage)
  const void* proj_w;         // projection [H][CpProjIn] (the kernels of a projected code predictor only)
  const uint16_t* proj_s;     // its scales (i8row: per row; i8g32: per 32 weights)
  const float* proj_b;        // its bias [H], nullable
};

// A code-predictor launch as the kernel takes it: the talker descriptor of the shared kernel (max_len = the positions,
// no processor) and the code predictor's own arguments. Pairing needs a position 1 to pair with (n_positions >= 2,
// checked by sk_cp_frame).
inline void cp_launch_args(const sk_cp_desc* d, sk_talker_desc& t, CpArgs& cp) {
  t = sk_talker_desc{};
  t.n_layers = d->n_layers; t.hidden = d->hidden; t.inter = d->inter; t.nq = d->nq; t.nkv = d->nkv;
  t.vocab = d->vocab; t.max_len = d->n_positions; t.wd = d->wd; t.ct = d->ct; t.eps = d->eps;
  t.layers = d->layers; t.norm = d->norm; t.rope = d->rope; t.id0 = const_cast<int64_t*>(d->id0);
  t.out = d->codes; t.rep_pen = 1.f; t.eos = -1; t.talker_processor = 0;
  t.logits = d->logits; t.layer_out = d->layer_out; t.workspace = d->workspace; t.workspace_bytes = d->workspace_bytes;
  t.do_sample = d->do_sample; t.inv_temp = d->inv_temp; t.top_k = d->top_k; t.seed = d->seed; t.counter = d->counter;
  cp = CpArgs{d->x0, d->emb, d->head_w, d->head_s, d->emb0_rows, d->pair ? 1 : 0, d->proj_w, d->proj_s, d->proj_b};
}

// Everything a role function needs about this workgroup and launch.
struct Ctx {
  sk_talker_desc d;
  CpArgs cp;
  void* ws;
  char* region;    // the cell region
  uint32_t slots;  // this XCD's page slot in each quarter of the region (3 bits per quarter)
  uint32_t x;     // XCD = kv head
  int r, g;       // rank in the XCD, global workgroup index
  uint32_t base, tpf;
  int pos0, n_frames, L;
  uint64_t seed, cnt0;  // sampled picks: Philox key and the draw counter at launch
  uint64_t* trace;  // per-stage timestamps of frame 0 (null when tracing is off)
  uint8_t dl[Ws::kHops];  // poll start delay of each exchange, sleep units
  __device__ void tr(int role, int f, int l, int ev) const {
    if (trace && f == 0 && l < Ws::kTraceLayers)
      trace[(((size_t)g * 2 + role) * Ws::kTraceLayers + l) * Ws::kTraceEvents + ev] = (uint64_t)wall_clock64();
  }
  __device__ uint64_t* tslot(int role, int f, int l, int ev) const {  // trace slot address, null when not traced
    return (trace && f == 0 && l < Ws::kTraceLayers)
               ? trace + (((size_t)g * 2 + role) * Ws::kTraceLayers + l) * Ws::kTraceEvents + ev
               : nullptr;
  }
  __device__ void tr_clk(int role, int f, int l, int ev) const {  // shader clock counter instead of wall clock
    if (trace && f == 0 && l < Ws::kTraceLayers)
      trace[(((size_t)g * 2 + role) * Ws::kTraceLayers + l) * Ws::kTraceEvents + ev] = (uint64_t)clock64();
  }
  __device__ uint32_t tick(int f, int l, int s) const {
    return base + 1u + (uint32_t)f * tpf + (uint32_t)l * 8u + (uint32_t)s;
  }

  __device__ const bf16_t* kh(const sk_layer_desc& Ly) const { return (const bf16_t*)Ly.kc + (size_t)x * d.max_len * SK_HD; }
  __device__ const bf16_t* vh(const sk_layer_desc& Ly) const { return (const bf16_t*)Ly.vc + (size_t)x * d.max_len * SK_HD; }
};

__device__ void fail(const Ctx& c, uint32_t code, int f, int l) {
  st_u32_dev(c.ws, Ws::kDiag, code);
  st_u32_dev(c.ws, Ws::kDiag + 4, (uint32_t)f);
  st_u32_dev(c.ws, Ws::kDiag + 8, (uint32_t)l);
  st_u32_dev(c.ws, Ws::kDiag + 12, (uint32_t)c.g);
  __builtin_amdgcn_s_waitcnt(0);
  st_u32_dev(c.ws, Ws::kErr, code);
}

// Compute wave cw's part of a sampled pick (steps 1-3 above), between the barrier that hands the control wave the
// processed logits and the one that ends the pick; it passes the same three barriers as the control wave. Out of
// line for the same reason as the control wave's part: inlined, its registers pushed the compute waves' layer loop
// into spills (38 against 1 spilled VGPRs on the 0.6B talker).
template <int V, int W, bool SINGLE = false>
__device__ __attribute__((noinline)) void pick_compute(uint32_t cb_, uint32_t ci_, uint32_t ck_, uint32_t ps_,
                                                       char* region_, uint32_t slots_,
                                                       void* ws_, uint32_t vals_, uint32_t e_, uint64_t draw_,
                                                       uint64_t seed_, int top_k_, uint32_t delay_, int f_, int L_,
                                                       int g_, int cw_, int lane, uint64_t* tp_) {
  constexpr int NB = V / 128;  // value cell pairs per lane over the whole vocabulary
  constexpr int NQ = NB / W;   // this wave's: pairs NQ cw .. NQ cw + NQ - 1, cells 2 lane + 128 b, + 1
  static_assert(W == 4 && NB % W == 0, "a quarter of the values per compute wave");
  lds_u32x4* cb = lds_at<lds_u32x4>(cb_);
  lds_u16* ci = lds_at<lds_u16>(ci_);
  lds_u32* ck = lds_at<lds_u32>(ck_);
  lds_pick* ps = lds_at<lds_pick>(ps_);
  char* region = uniform(region_);
  const uint32_t slots = __builtin_amdgcn_readfirstlane(slots_);
  void* ws = uniform(ws_);
  const uint32_t vals = __builtin_amdgcn_readfirstlane(vals_), e = __builtin_amdgcn_readfirstlane(e_);
  const uint32_t d0 = __builtin_amdgcn_readfirstlane((uint32_t)draw_), d1 = __builtin_amdgcn_readfirstlane((uint32_t)(draw_ >> 32));
  const uint32_t k0 = __builtin_amdgcn_readfirstlane((uint32_t)seed_), k1 = __builtin_amdgcn_readfirstlane((uint32_t)(seed_ >> 32));
  const uint64_t draw = ((uint64_t)d1 << 32) | d0;
  const int top_k = __builtin_amdgcn_readfirstlane(top_k_);
  const uint32_t delay = __builtin_amdgcn_readfirstlane(delay_);
  const int f = __builtin_amdgcn_readfirstlane(f_), L = __builtin_amdgcn_readfirstlane(L_);
  const int g = __builtin_amdgcn_readfirstlane(g_), cw = __builtin_amdgcn_readfirstlane(cw_);
  gptr<uint64_t> tp = (gptr<uint64_t>)uniform(tp_);  // wave 0's wall-clock stamps when tracing (tp[0..7]), else null
  const int b0 = NQ * cw;
  auto gather = [&]() {
#pragma unroll
    for (int b = 0; b < NQ; b++) {
      const uint32_t so = __builtin_amdgcn_readfirstlane(read_off<SINGLE>(slots, vals + 128u * (uint32_t)(b0 + b)));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(region), (lds_void*)(cb + 64 * (b0 + b)), 16,
                                               (uint32_t)lane * 16u, so, 0, kPolDev);
    }
  };
  sleep_units(delay);
  gather();
  uint64_t st[8] = {};  // stamps, stored at the end (a global store in flight would hold up the next wait)
  const bool trc = tp != nullptr;
  if (trc) st[0] = (uint64_t)wall_clock64();
  bool good = false;
  uint32_t spins = 0;
  for (uint32_t spin = 0;; spin++) {
    spins = spin;
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the direct loads have landed in LDS
    bool ok = true;
#pragma unroll
    for (int b = 0; b < NQ; b++) {
      const u32x4 q = cb[64 * (b0 + b) + lane];
      ok &= q.y == e && q.w == e;
    }
    if (__all(ok)) { good = true; break; }
    if ((spin & 63) == 63) {
      if (ld_u32_dev(ws, Ws::kErr) != 0) break;
      if (spin > kSpinLimit) {  // the error word and the diagnostic words, as fail() writes them
        if (lane == 0) {
          st_u32_dev(ws, Ws::kDiag, 20u);
          st_u32_dev(ws, Ws::kDiag + 4, (uint32_t)f);
          st_u32_dev(ws, Ws::kDiag + 8, (uint32_t)L);
          st_u32_dev(ws, Ws::kDiag + 12, (uint32_t)g);
          __builtin_amdgcn_s_waitcnt(0);
          st_u32_dev(ws, Ws::kErr, 20u);
        }
        break;
      }
    }
    __builtin_amdgcn_s_sleep(1);
    gather();
  }
  if (!good && lane == 0) __hip_atomic_fetch_or(&ps->bad, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  if (trc) { st[1] = (uint64_t)wall_clock64(); st[2] = spins; }
  wg_sync();  // (1)
  if (trc) st[3] = (uint64_t)wall_clock64();
  const bool bad = __builtin_amdgcn_readfirstlane(ps->bad) != 0;
  if (!bad) {
    const uint32_t lb = __builtin_amdgcn_readfirstlane(ps->lb);
    uint32_t key[2 * NQ];
    uint32_t cnt = 0;
#pragma unroll
    for (int b = 0; b < NQ; b++) {
      const u32x4 q = cb[64 * (b0 + b) + lane];
      key[2 * b] = order_key(__uint_as_float(q.x));
      key[2 * b + 1] = order_key(__uint_as_float(q.z));
      cnt += (uint32_t)(key[2 * b] >= lb) + (uint32_t)(key[2 * b + 1] >= lb);
    }
    const uint32_t incl = wave_incl_scan_u32(cnt);
    uint32_t base = 0;
    if (lane == 63) base = __hip_atomic_fetch_add(&ps->n, incl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    uint32_t at = (uint32_t)__builtin_amdgcn_readlane((int)base, 63) + incl - cnt;
#pragma unroll
    for (int b = 0; b < NQ; b++) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        if (key[2 * b + h] >= lb) {
          ci[at] = (uint16_t)(2 * lane + 128 * (b0 + b) + h);
          ck[at] = key[2 * b + h];
          at++;
        }
      }
    }
  }
  if (trc) st[4] = (uint64_t)wall_clock64();
  wg_sync();  // (2)
  const uint32_t n = __builtin_amdgcn_readfirstlane(ps->n);
  if (trc) st[5] = (uint64_t)wall_clock64();
  if (!bad && top_k > 0 && top_k <= 64 && top_k < V && n <= 256u) {
    // G lanes per candidate (consecutive lanes of a quad), each counting the larger keys in every G-th group of
    // four; a lane that holds no candidate counts nothing
    const uint32_t sh = n <= 64u ? 2u : n <= 128u ? 1u : 0u, G = 1u << sh;
    const uint32_t t = (uint32_t)(64 * cw + lane), j = t >> sh, part = t & (G - 1u);
    const bool has = j < n;
    const uint32_t key = has ? ck[j] : 0xffffffffu;
    const lds_u32x4* ck4 = (const lds_u32x4*)ck;
    const bool wv = ((uint32_t)(64 * cw) >> sh) < n;  // this wave holds candidates
    const uint32_t nf = wv ? n / 4 : 0u;                // full groups of four
    uint32_t gt = 0;
    const uint32_t nit = (nf + G - 1u) >> sh;  // a trip count common to the wave, so the reads overlap
#pragma unroll 4
    for (uint32_t it = 0; it < nit; it++) {
      const uint32_t q = (it << sh) + part;
      const u32x4 k4 = ck4[q < nf ? q : 0u];
      const uint32_t c4 = (uint32_t)(k4.x > key) + (uint32_t)(k4.y > key) + (uint32_t)(k4.z > key) + (uint32_t)(k4.w > key);
      gt += q < nf ? c4 : 0u;
    }
    if (wv && part == 0)
      for (uint32_t i = n & ~3u; i < n; i++) gt += (uint32_t)(ck[i] > key);
    if (sh >= 1) gt += dppu<0xB1>(gt);  // quad_perm [1,0,3,2]: the pair's sum
    if (sh >= 2) gt += dppu<0x4E>(gt);  // quad_perm [2,3,0,1]: the quad's
    if (trc) st[6] = (uint64_t)wall_clock64();
    const bool kept = has && part == 0 && gt < (uint32_t)top_k && key != kNegInfKey;  // key >= threshold, not -inf
    float best = -INFINITY;
    uint32_t bi = 0x7fffffffu;
    if (kept) {
      const uint32_t i = ci[j];
      const float gv = gumbel(key_value(key), i, draw, k0, k1);
      if (gv == gv) { best = gv; bi = i; }  // a NaN never wins
    }
    const float gmax = wave_max(best);
    const uint32_t pick = ~wave_max_u32(best == gmax ? ~bi : 0u);
    const uint32_t nk = (uint32_t)__popcll(__ballot(kept));
    if (lane == 0) { ps->gv[cw] = gmax; ps->bi[cw] = pick; ps->nk[cw] = nk; }
    if (trc) st[7] = (uint64_t)wall_clock64();
  }
  wg_sync();  // (3)
  if (trc && lane == 0) {
#pragma unroll
    for (int k = 0; k < 8; k++) tp[k] = st[k];
  }
}

// Barriers of the attention stage after its input has arrived (both roles execute the same count): one after
// the q / k / v preparation, then with a non-empty chunk one after the scores (P V is published by dimension slice
// from registers, with no barrier after it).
template <class Ck>
__device__ __forceinline__ int attn_barriers(const Ck& ck) { return 1 + (ck.n > 0 ? 1 : 0); }

// ================================================================================================================
// Control wave
// ================================================================================================================
// Control wave of the code predictor's paired first pass (positions 0 and 1 as two rows per stage, the
// reference's cp_pair: qwen3/kernels.py:276-310, 600-617). The control wave polls and stages the first row's inputs
// as in a regular frame; the compute waves poll the second row's from its own cells (b1, b3..b6) at the same time (two
// polls in parallel instead of one after the other), and compute both rows' attention (two barriers). Returns
// false when a poll of either row failed (P.bad, or the stage flags for the compute waves).
template <int H, int I, int W, int V, bool CP>
__device__ __forceinline__ bool ctl_pair_pass(const Ctx& c, Lds<H, I, W, V, CP>& S, int lane) {
  constexpr int kNP = H / 128;
  constexpr bool kLO = true;  // lane offsets, as the compute waves of the pass use them
  static_assert(W == 4, "the paired pass stages its inputs from registers");
  const Layout LY(H, I);
  LdsPair<H, I>& P = *(LdsPair<H, I>*)((char*)&S + sizeof(Lds<H, I, W, V, CP>));
  const float eps = c.d.eps;
  const int f = 0;
  for (int l = 0; l < c.L; l++) {
    const sk_layer_desc& Ly = S.desc[l];
    bool ok = true;
    float ss;
    {
      // S1 input: position 0's vector (layer 0), else the residual, times the input norm
      float2 w[kNP], v[kNP];
      load_pairs<kNP>(Ly.in_norm, w, lane);
      if (l == 0) {
        load_pairs<kNP>(c.cp.x0, v, lane);
      } else {
        after_publish(S, (uint32_t)l * 4u, c.dl[Ws::kHopS1]);
        u32x4 q[kNP];
        ok = poll_regs<kNP, kLO>(c.region, c.slots, LY.e6, c.tick(f, l - 1, 5), q, c.ws, lane, c, 11u, f, l);
        cells_to_pairs<kNP>(q, v);
      }
      ss = stage_rms<kNP>(v, w, S.hin, S.xs[0], lane);
    }
    if (lane == 0) { S.inv = rsqrtf(ss / H + eps); S.flags[0] = !ok; }
    wg_sync();
    if (!ok || P.bad) return false;
    // S2 input: q|k|v of this workgroup's head
    after_publish(S, (uint32_t)l * 4u + 1u, c.dl[Ws::kHopS2]);
    ok = poll_cells<mb(512), false, kLO>(c.region, c.slots, LY.e1, 512, c.tick(f, l, 0), S.qkv, c.ws, lane, c, 12u, f, l);
    if (lane == 0) S.flags[1] = !ok;
    wg_sync();
    if (!ok || P.bad) return false;
    wg_sync();  // paired attention: vectors ready
    wg_sync();  // paired attention: scores of the second row
    // S4 input: the attention output, written whole by the workgroups themselves
    sleep_units(c.dl[Ws::kHopS4]);
    ok = poll_cells<mb(kQ), true, kLO>(c.region, c.slots, LY.e3, kQ, c.tick(f, l, 2), S.xs[1], c.ws, lane, c, 14u, f, l);
    if (lane == 0) S.flags[2] = !ok;
    wg_sync();
    if (!ok || P.bad) return false;
    {
      // S5 input: the residual after o, times the post-attention norm
      float2 w[kNP], v[kNP];
      load_pairs<kNP>(Ly.post_norm, w, lane);
      after_publish(S, (uint32_t)l * 4u + 2u, c.dl[Ws::kHopS5]);
      u32x4 q[kNP];
      ok = poll_regs<kNP, kLO>(c.region, c.slots, LY.e4, c.tick(f, l, 3), q, c.ws, lane, c, 15u, f, l);
      cells_to_pairs<kNP>(q, v);
      ss = stage_rms<kNP>(v, w, S.hmid, S.xs[0], lane);
    }
    if (lane == 0) { S.inv = rsqrtf(ss / H + eps); S.flags[3] = !ok; }
    wg_sync();
    if (!ok || P.bad) return false;
    // S6 input: the SwiGLU activation
    after_publish(S, (uint32_t)l * 4u + 3u, c.dl[Ws::kHopS6]);
    ok = poll_cells<mbh(I), true, kLO>(c.region, c.slots, LY.e5, I, c.tick(f, l, 4), S.xs[1], c.ws, lane, c, 16u, f, l);
    if (lane == 0) S.flags[4] = !ok;
    wg_sync();
    if (!ok || P.bad) return false;
  }
  return true;
}

template <int H, int I, int W, int V, bool CP, bool SMP, bool F16 = false, bool SG = false>
__device__ void run_control(const Ctx& c, Lds<H, I, W, V, CP>& S, int lane) {
  // The RMSNorm inputs are polled into registers and staged from there (kNP element pairs per lane)
  constexpr int kNP = H / 128;
  constexpr int PK = CP ? CpProjIn<H, I>::value : 0;
  // Stage publications per position: 4 per layer, and with a projection one more at the start of each position
  // (the waits below count 4 (fq L + l) + k, plus kP0 (fq + 1))
  constexpr uint32_t kP0 = PK > 0 ? 1u : 0u;
  constexpr bool kLO = LaneOffsetPolls<H>::value;
  const Layout LY(H, I);
  const float eps = c.d.eps;
  const bf16_t* emb = (const bf16_t*)c.d.emb;
  // code predictor: lane f holds position f's embedding table (read once; per position it was a memory round trip
  // ahead of the row's own)
  const uint64_t emb_l = (CP && lane < c.d.max_len) ? (uint64_t)gload(c.cp.emb + lane) : 0;
  int64_t tok = gload(c.d.id0);
  if (CP && c.g == 0 && lane == 0 && c.d.out) gstore(c.d.out, tok);  // code 0 passes through
  // After the code predictor's paired pass (positions 0 and 1, a launch of its own: k_frames with PAIRK) frame 1
  // runs only its head, from the pass's second row, and the stage publications of this launch start at frame 2
  // (fq counts the frames with layers before this one).
  const bool pr = CP && c.cp.pair;
  for (int f = pr ? 1 : 0; f < c.n_frames; f++) {
    const int pos = c.pos0 + f;
    const auto ck = make_chunk<CP>(pos, c.r, Cfg<H, I, W, V, CP>::whole(pos));
    const int fq = pr ? f - 2 : f;
    for (int l = 0; l < (pr && f == 1 ? 0 : c.L); l++) {
      const sk_layer_desc& Ly = S.desc[l];
      bool ok = true;
      float ss = 0.f;
      {
        // S1 input from registers: embedding row (layer 0) or the previous layer's residual (polled), times the
        // input norm; lane holds elements 2 lane + 128 b, + 1
        float2 w[kNP], v[kNP];
        load_pairs<kNP>(Ly.in_norm, w, lane);
        if (lane == 0) c.tr(0, f, l, 0);
        if (CP && PK > 0 && l == 0) {
          // S0, the projection: its input (x0 at position 0, else the embedding row of the previous code; PK wide)
          // staged plainly for the compute waves' dot, then the projected vector polled as the stack's input
          constexpr int kNPP = PK > 0 ? PK / 128 : 1;
          float2 x[kNPP];
          if (f == 0) {
            load_pairs<kNPP>(c.cp.x0, x, lane);
          } else {
            const bf16_t* tab = (const bf16_t*)lane_u64(emb_l, f);
#pragma unroll
            for (int b = 0; b < kNPP; b++) {
              const uint32_t u = gload((const uint32_t*)(tab + (size_t)tok * PK) + lane + 64 * b);
              x[b] = make_float2(bf2f(u & 0xffffu), bf2f(u >> 16));
            }
          }
          stage_plain<kNPP>(x, S.xs[0], lane);
          wg_sync();
          after_publish(S, (uint32_t)(fq * c.L) * 4u + kP0 * (uint32_t)(fq + 1), c.dl[Ws::kHopS1]);
          u32x4 q[kNP];
          ok = poll_regs<kNP, kLO, SG>(c.region, c.slots, LY.pj, c.tick(f, 0, 6), q, c.ws, lane, c, 10u, f, l);
          cells_to_pairs<kNP>(q, v);
        } else if (l == 0) {
          if (CP && f == 0) {
            load_pairs<kNP>(c.cp.x0, v, lane);
          } else if (!CP && c.d.in_groups > 0) {
            // talker_in: the embedding rows of the frame's codes summed in group order, then the pad row. Lane g
            // reads group g's table address and code, so the rows' loads of 4 groups at a time go out together
            // (one group after the other cost two dependent memory round trips per group).
            const int ng = c.d.in_groups;
            const uint64_t tl = lane < ng ? gload(c.d.in_tabs + lane) : 0;
            const int64_t cl = lane < ng ? gload(c.d.in_codes + lane) : 0;
#pragma unroll
            for (int b = 0; b < kNP; b++) v[b] = make_float2(0.f, 0.f);
            for (int g0 = 0; g0 < ng; g0 += 4) {
              uint32_t u[4][kNP];
#pragma unroll
              for (int j = 0; j < 4; j++) {
                const int gi = min(g0 + j, ng - 1);
                const bf16_t* tab = (const bf16_t*)lane_u64(tl, gi);
                const int64_t code = (int64_t)lane_u64((uint64_t)cl, gi);
#pragma unroll
                for (int b = 0; b < kNP; b++) u[j][b] = gload((const uint32_t*)(tab + (size_t)code * H) + lane + 64 * b);
              }
#pragma unroll
              for (int j = 0; j < 4; j++) {
                if (g0 + j < ng) {
#pragma unroll
                  for (int b = 0; b < kNP; b++) {
                    v[b].x += bf2f(u[j][b] & 0xffffu);
                    v[b].y += bf2f(u[j][b] >> 16);
                  }
                }
              }
            }
#pragma unroll
            for (int b = 0; b < kNP; b++) {
              const uint32_t u = gload((const uint32_t*)c.d.in_pad + lane + 64 * b);
              v[b].x += bf2f(u & 0xffffu);
              v[b].y += bf2f(u >> 16);
            }
          } else {
            const bf16_t* tab = CP ? (const bf16_t*)lane_u64(emb_l, f) : emb;
#pragma unroll
            for (int b = 0; b < kNP; b++) {
              const uint32_t u = gload((const uint32_t*)(tab + (size_t)tok * H) + lane + 64 * b);
              v[b] = make_float2(bf2f(u & 0xffffu), bf2f(u >> 16));
            }
          }
        } else {
          after_publish(S, (uint32_t)(fq * c.L + l) * 4u + kP0 * (uint32_t)(fq + 1), c.dl[Ws::kHopS1]);  // own part of the previous layer's down output
          u32x4 q[kNP];
          ok = poll_regs<kNP, kLO, SG>(c.region, c.slots, LY.e6, c.tick(f, l - 1, 5), q, c.ws, lane, c, 11u, f, l);
          cells_to_pairs<kNP>(q, v);
        }
        ss = stage_rms<kNP>(v, w, S.hin, S.xs[0], lane);
      }
      if (lane == 0) { S.inv = rsqrtf(ss / H + eps); S.flags[0] = !ok; c.tr(0, f, l, 1); }
      wg_sync();
      if (!ok) return;
      // S2 input: this head's q/k/v
      after_publish(S, (uint32_t)(fq * c.L + l) * 4u + 1u + kP0 * (uint32_t)(fq + 1), c.dl[Ws::kHopS2]);
      ok = poll_cells<mb(512), false, kLO>(c.region, c.slots, LY.e1, 512, c.tick(f, l, 0), S.qkv, c.ws, lane, c, 12u, f, l);
      if (lane == 0) { S.flags[1] = !ok; c.tr(0, f, l, 2); }
      wg_sync();
      if (!ok) return;
      for (int b = 0; b < (CP && F16 ? 1 : attn_barriers(ck)); b++) wg_sync();
      if (lane == 0) c.tr(0, f, l, 3);
      // S3: merge of the 32 chunk partials for q head 2x + r/16, dims [8 (r % 16), 8 (r % 16) + 8)
      {
        const uint32_t e = c.tick(f, l, 1);
        const int mh = c.r >> 4, md0 = 8 * (c.r & 15);
        if (!ck.whole) {  // whole-cache attention publishes the S4 input itself
          sleep_units(c.dl[Ws::kHopS3]);  // the compute waves publish their partial after the last attention barrier (and P V)
          // lane = chunk + 32 * half: lane polls its chunk's (m, l) of head mh and the 4 dims md0 + 4 half .. + 3 of
          // its o slice straight into registers (both halves read the same (m, l)), so the merge needs no LDS
          static_assert(kChunks == 32, "merge lane mapping");
          const int ch = lane & 31, hh = lane >> 5;
          const uint32_t om = own_off(c.slots, LY.e2m + 4 * ch + 2 * mh);
          const uint32_t oo = own_off(c.slots, LY.e2o + 2 * SK_HD * ch + mh * SK_HD + md0 + 4 * hh);
          const __amdgpu_buffer_rsrc_t rc = make_rsrc(c.region);
          u32x4 ml, oa, ob;
          for (uint32_t spin = 0;; spin++) {
            ml = __builtin_amdgcn_raw_buffer_load_b128(rc, om, 0, kPolDev);
            oa = __builtin_amdgcn_raw_buffer_load_b128(rc, oo, 0, kPolDev);
            ob = __builtin_amdgcn_raw_buffer_load_b128(rc, oo + 16u, 0, kPolDev);
            if (__all(ml.y == e && ml.w == e && oa.y == e && oa.w == e && ob.y == e && ob.w == e)) break;
            if ((spin & 63) == 63) {
              if (ld_u32_dev(c.ws, Ws::kErr) != 0) { ok = false; break; }
              if (spin > kSpinLimit) { if (lane == 0) fail(c, 13u, f, l); ok = false; break; }
            }
            __builtin_amdgcn_s_sleep(1);
          }
          if (lane == 0) c.tr(0, f, l, 8);
          if (ok) {
            // one exp per chunk; each half sums its 32 lanes (rows 0 + 1, rows 2 + 3), so lanes 16 and 48 end with
            // the weight sum and the 4 merged dims of their half (empty chunks carry m = -inf and weigh nothing)
            const float mc = __uint_as_float(ml.x);
            const float rm = row16_max(mc);
            const float M = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 0)),
                                  __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rm), 16)));
            const float fct = mc == -INFINITY ? 0.f : expf(mc - M);
            float v[5] = {fct * __uint_as_float(ml.z), fct * __uint_as_float(oa.x), fct * __uint_as_float(oa.z),
                          fct * __uint_as_float(ob.x), fct * __uint_as_float(ob.z)};
#pragma unroll
            for (int d = 0; d < 5; d++) {
              v[d] = row16_sum(v[d]);
              v[d] += dpp<0x142, 0xA>(v[d]);  // row_bcast:15 into rows 1 and 3
            }
            if (ch == 16) {  // lanes 16 and 48: the sums of their half, stored into every copy
              const float Lw = v[0];
              const uint32_t o0 = LY.e3 + (2 * c.x + mh) * SK_HD + md0 + 4 * hh, e3 = c.tick(f, l, 2);
              put2_all<SG>(c.region, o0, Lw > 0.f ? v[1] / Lw : 0.f, Lw > 0.f ? v[2] / Lw : 0.f, e3);
              put2_all<SG>(c.region, o0 + 2, Lw > 0.f ? v[3] / Lw : 0.f, Lw > 0.f ? v[4] / Lw : 0.f, e3);
            }
          }
        }
        sleep_units(c.dl[Ws::kHopS4]);  // S4 input: the merges of all workgroups, this one's included
        if (lane == 0) c.tr(0, f, l, 4);
      }
      // S4 input: the whole attention output
      ok = ok && poll_cells<mb(kQ), true, kLO, SG>(c.region, c.slots, LY.e3, kQ, c.tick(f, l, 2), S.xs[1], c.ws, lane, c, 14u, f, l);
      if (lane == 0) { S.flags[2] = !ok; c.tr(0, f, l, 5); }
      wg_sync();
      if (!ok) return;
      // S5 input: residual after o, times the post-attention norm (loaded while the exchange is under way)
      {
        float2 w[kNP], v[kNP];
        load_pairs<kNP>(Ly.post_norm, w, lane);
        after_publish(S, (uint32_t)(fq * c.L + l) * 4u + 2u + kP0 * (uint32_t)(fq + 1), c.dl[Ws::kHopS5]);
        u32x4 q[kNP];
        ok = poll_regs<kNP, kLO, SG>(c.region, c.slots, LY.e4, c.tick(f, l, 3), q, c.ws, lane, c, 15u, f, l);
        cells_to_pairs<kNP>(q, v);
        ss = stage_rms<kNP>(v, w, S.hmid, S.xs[0], lane);
      }
      if (lane == 0) { S.inv = rsqrtf(ss / H + eps); S.flags[3] = !ok; c.tr(0, f, l, 6); }
      wg_sync();
      if (!ok) return;
      // S6 input: the whole SwiGLU activation
      after_publish(S, (uint32_t)(fq * c.L + l) * 4u + 3u + kP0 * (uint32_t)(fq + 1), c.dl[Ws::kHopS6]);
      ok = poll_cells<mbh(I), true, kLO, SG>(c.region, c.slots, LY.e5, I, c.tick(f, l, 4), S.xs[1], c.ws, lane, c, 16u, f, l);
      if (lane == 0) { S.flags[4] = !ok; c.tr(0, f, l, 7); }
      wg_sync();
      if (!ok) return;
    }
    if (CP && f == 0) continue;  // the code predictor's position 0 has no head
    // head input: final residual times the final norm
    bool ok;
    float ss = 0.f;
    {
      float2 w[kNP], v[kNP];
      load_pairs<kNP>(c.d.norm, w, lane);
      after_publish(S, (uint32_t)((fq + 1) * c.L) * 4u + kP0 * (uint32_t)(fq + 1), c.dl[Ws::kHopHead]);
      u32x4 q[kNP];
      // the head of frame 1 after a paired pass reads the pass's second row
      const bool hb = pr && f == 1;
      ok = poll_regs<kNP, kLO, SG>(c.region, c.slots, hb ? LY.b6 : LY.e6, c.tick(hb ? 0 : f, c.L - 1, 5), q, c.ws, lane, c,
                               17u, f, c.L);
      cells_to_pairs<kNP>(q, v);
      ss = stage_rms<kNP>(v, w, S.hin, S.xs[0], lane);
      if (lane == 0) { S.inv = rsqrtf(ss / H + eps); S.flags[5] = !ok; }
      if (!CP && c.d.final_out && c.g == 0 && ok) {  // the final norm's output, h * inv * w (rmsnorm)
        const float inv = rsqrtf(ss / H + eps);
#pragma unroll
        for (int b = 0; b < kNP; b++)
        {
          gstore(c.d.final_out + 2 * lane + 128 * b, (v[b].x * inv) * w[b].x);
          gstore(c.d.final_out + 2 * lane + 128 * b + 1, (v[b].y * inv) * w[b].y);
        }
      }
    }
    wg_sync();
    if (!ok) return;
    wg_sync();  // candidates (greedy) or processed logits (sampled) of the compute waves are in S.cand / S.hv
    if (SMP && lane == 0) c.tr(0, f, c.L, 9);
    if constexpr (SMP) {
      // every workgroup publishes its processed logits and draws the same pick from all of them, the control wave
      // with the compute waves (pick_compute)
      // S.xs[0] and S.xs[1] are free here (the head dot has consumed its input and the next frame's inputs
      // are staged after the pick): candidate indices and keys
      static_assert(V <= Lds<H, I, W, V, CP>::XS, "candidate keys fit a staging buffer");
      const int64_t t = sampled_pick<V, V / kWG, SG>(c.region, c.slots, LY.e8, LY.e7, c.g, c.tick(f, c.L, 1), lds_addr(S.hv),
                                                 lds_addr((char*)&S + kPickCopy<H, I, W, V, CP>), lds_addr(S.xs[0]),
                                                 lds_addr(S.xs[1]), lds_addr((char*)&S + kPickShared<H, I, W, V, CP>),
                                                 c.d.top_k, c.cnt0 + (uint64_t)(CP ? f - 1 : f),
                                                 c.seed, c.ws, c.dl[Ws::kHopPick], lane, c.tslot(0, f, c.L, 0));
      ok = t >= 0;
      if (ok) tok = t;
      else if (t == -2 && lane == 0) fail(c, 19u, f, c.L);
      if (lane == 0) { S.tok = tok; S.flags[6] = !ok; }
    } else {
    {
      uint64_t best = 0;
      for (int i = 0; i < W; i++) best = S.cand[i] > best ? S.cand[i] : best;
      const uint32_t e = c.tick(f, c.L, 0);
      put2_lanes<SG>(c.region, LY.e7 + 2 * c.g, __uint_as_float((uint32_t)(best >> 32)), __uint_as_float((uint32_t)best),
                 e, lane);
    }
    // pick: reduce the 256 candidates
    {
      const uint32_t e = c.tick(f, c.L, 0);
      sleep_units(c.dl[Ws::kHopPick]);
      uint64_t best = 0;
      for (uint32_t spin = 0;; spin++) {
        bool good = true;
        best = 0;
        u32x4 q[kWG / 64];
#pragma unroll
        for (int j = 0; j < kWG / 64; j++) q[j] = get2<SG>(c.region, c.slots, LY.e7 + 2 * (lane + 64 * j));
#pragma unroll
        for (int j = 0; j < kWG / 64; j++) {
          good &= q[j].y == e && q[j].w == e;
          const uint64_t k = ((uint64_t)q[j].x << 32) | q[j].z;
          best = k > best ? k : best;
        }
        if (__all(good)) break;
        if ((spin & 63) == 63) {
          if (ld_u32_dev(c.ws, Ws::kErr) != 0) { ok = false; break; }
          if (spin > kSpinLimit) { if (lane == 0) fail(c, 18u, f, c.L); ok = false; break; }
        }
        __builtin_amdgcn_s_sleep(1);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const uint64_t b = __shfl_xor(best, o);
        best = b > best ? b : best;
      }
      tok = best ? (int64_t)(0xffffffffu - (uint32_t)best) : 0;
      if (lane == 0) { S.tok = tok; S.flags[6] = !ok; }
    }
    }
    if (SMP && lane == 0) c.tr(0, f, c.L, 15);
    wg_sync();
    if (!ok) return;
    if (c.g == 0 && lane == 0) {
      // device-side frame state, as the sampler leaves it (qwen3/sampler.py:147-156)
      if (c.d.out) gstore(c.d.out + f, tok);
      if (c.d.seen) {
        // read back by later frames of this launch through device-coherent loads
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)1, make_rsrc(uniform(c.d.seen)), (uint32_t)tok, 0, kPolDev);
        __builtin_amdgcn_s_waitcnt(0);
      }
    }
  }
  if (!CP && c.g == 0 && lane == 0) {
    if (ld_u32_dev(c.ws, Ws::kErr) == 0) {
      gstore(c.d.id0, tok);
      if (c.d.next_id0) gstore(c.d.next_id0, tok);
      gstore(c.d.pos, (int64_t)(c.pos0 + c.n_frames));
      if (c.d.ngen) gstore(c.d.ngen, gload(c.d.ngen) + (int64_t)c.n_frames);
    }
  }
  if (SMP && c.g == 0 && lane == 0 && ld_u32_dev(c.ws, Ws::kErr) == 0)
    gstore(c.d.counter, c.cnt0 + (uint64_t)(CP ? c.n_frames - 1 : c.n_frames));
}

// ================================================================================================================
// Compute waves
// ================================================================================================================
// Compute waves of the code predictor's paired first pass (positions 0 and 1 as two rows per stage;
// ctl_pair_pass is the control wave's side), run before the frame loop and before run_compute sets up its own
// state (weights, rows, RoPE): nothing of this pass stays live into the loop, whose registers are then allocated
// as without it. The layer weights in registers serve both rows' dots, and the attention covers the two new
// positions (the first row attends to position 0 alone, the second to both). The compute waves also poll and stage
// the second row's inputs while the control wave polls the first row's: wave 3 the residuals (with their RMSNorm),
// wave 2 the q|k|v, waves 0-1 the attention output and waves 0-2 the activation, 1024 cells each. Frame 1 then
// runs only its head. Returns false when a poll failed.
template <int H, int I, int W, int V, bool CP, int WD, bool KEEP>
__device__ __forceinline__ bool compute_pair(const Ctx& c, Lds<H, I, W, V, CP>& S, int cw, int tid, int lane) {
  using C = CfgW<H, I, W, V, CP, WD>;
  // lane offsets for every cell and weight access: per-load vector addresses, hoisted out of the layer loop by the
  // compiler, held ~100 registers through the pass and made it spill
  constexpr bool kLO = true;
  constexpr int kNP = H / 128;
  static_assert(2 * 16 <= 64 && 2 * C::R_O <= 64 && C::R_GU <= 64 && 2 * C::R_D <= 64, "both rows fit S.pub");
  static_assert(kQ % 1024 == 0 && I % 1024 == 0 && kQ / 1024 <= W && I / 1024 <= W && W == 4,
                "the second row's polls: 1024-cell blocks, one per compute wave");
  const Layout LY(H, I);
  LdsPair<H, I>& P = *(LdsPair<H, I>*)((char*)&S + sizeof(Lds<H, I, W, V, CP>));
  const float eps = c.d.eps;
  const int x = (int)c.x, r = c.r, g = c.g;
  const int f = 0;
  // this wave's rows in every stage, as run_compute assigns them
  const int qkv_row0 = r < 16 ? 256 * x + 16 * r : r < 24 ? kQ + 128 * x + 16 * (r - 16) : kQ + kNKV * 128 + 128 * x + 16 * (r - 24);
  const int q_w0 = qkv_row0 + C::RW_QKV * cw;
  const int o_w0 = C::R_O * g + C::RW_O * cw, o_wn = max(0, min(C::RW_O, C::R_O - C::RW_O * cw));
  const int gu_w0 = C::R_GU * g + C::RW_GU * cw;
  const int d_w0 = C::R_D * g + C::RW_D * cw, d_wn = max(0, min(C::RW_D, C::R_D - C::RW_D * cw));
  static_assert(C::RW_O * W == C::R_O && C::RW_D * W == C::R_D, "every wave has rows of o and down");
  const int p = tid >> 7, dd = tid & 127;  // the attention's head and dim of this thread
  uint4 wq[C::RW_QKV][C::CH], wo[C::RW_O][C::CQ], wg[C::RW_GU][C::CH], wd[C::RW_D][C::CI];
  uint16_t sq[C::RW_QKV], so[C::RW_O], sg[C::RW_GU], sd[C::RW_D];
  constexpr bool G32 = WD == SK_WD_I8G32;  // i8g32: raw fp16 group scales, one per row and chunk
  uint16_t gq[G32 ? C::RW_QKV : 1][G32 ? C::CH : 1], go[G32 ? C::RW_O : 1][G32 ? C::CQ : 1];
  uint16_t gg[G32 ? C::RW_GU : 1][G32 ? C::CH : 1], gd[G32 ? C::RW_D : 1][G32 ? C::CI : 1];
  float a_cs, a_sn, a_n0, a_n1;  // RoPE of position 0 and the q / k norm weights of this wave's vector
  auto load_attn_vec = [&](const sk_layer_desc& Lx) {
    const float* nw = (cw & 3) == 2 ? Lx.kn : Lx.qn;
    a_cs = gload(c.d.rope + (size_t)c.pos0 * SK_HD + lane);
    a_sn = gload(c.d.rope + (size_t)c.pos0 * SK_HD + 64 + lane);
    a_n0 = gload(nw + lane);
    a_n1 = gload(nw + 64 + lane);
  };
  if (cw == 0 && lane == 0) P.bad = 0;
  // the second row's RMSNorm input from registers: P.hin / P.hmid, P.xs[0] and P.inv, as the control wave stages
  // the first row's
  auto stage_b = [&](const float2 (&v)[kNP], const float* nw, float* res) {
    float2 w[kNP];
    load_pairs<kNP>(nw, w, lane);
    const float ss = stage_rms<kNP>(v, w, res, P.xs[0], lane);
    if (lane == 0) P.inv = rsqrtf(ss / H + eps);
  };
  {
    const sk_layer_desc& L0 = S.desc[0];
    load_w<WD, C::RW_QKV, C::CH, kLO, KEEP>(wq, sq, gq, (const int8_t*)L0.qkv_w, L0.qkv_s, q_w0, C::RW_QKV, H, lane);
    load_attn_vec(L0);
    load_w<WD, C::RW_O, C::CQ, kLO, KEEP>(wo, so, go, (const int8_t*)L0.o_w, L0.o_s, o_w0, o_wn, kQ, lane);
  }
  __builtin_amdgcn_s_waitcnt(0);
  for (int l = 0; l < c.L; l++) {
    const sk_layer_desc& Ly = S.desc[l];
    // the next layer's weights are prefetched unconditionally (after the last layer the frame loop's prologue
    // loads frame 2's)
    const sk_layer_desc& Ln = S.desc[l == c.L - 1 ? 0 : l + 1];
    if (cw == 3) {  // the second row's S1 input: the talker embedding row of code 0 (layer 0), else its residual
      float2 v[kNP];
      if (l == 0) {
        const bf16_t* tab = (const bf16_t*)uniform(gload(c.cp.emb + 1));
        const int64_t tok = gload(c.d.id0);
#pragma unroll
        for (int b = 0; b < kNP; b++) {
          const uint32_t u = gload((const uint32_t*)(tab + (size_t)tok * H) + lane + 64 * b);
          v[b] = make_float2(bf2f(u & 0xffffu), bf2f(u >> 16));
        }
      } else {
        sleep_units(c.dl[Ws::kHopS1]);
        u32x4 q[kNP];
        const bool ok = poll_regs<kNP, kLO>(c.region, c.slots, LY.b6, c.tick(f, l - 1, 5), q, c.ws, lane, c, 11u, f, l);
        if (!ok && lane == 0) P.bad = 1;
        cells_to_pairs<kNP>(q, v);
      }
      stage_b(v, Ly.in_norm, P.hin);
    }
    // ---- S1: qkv rows of both positions
    wg_sync();
    if (S.flags[0] || P.bad) return false;
    {
      float ya[C::RW_QKV], yb[C::RW_QKV];
      dot2_w<WD, C::RW_QKV, C::CH>(wq, gq, S.xs[0], P.xs[0], lane, ya, yb);
      const float ia = S.inv, ib = P.inv;
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < C::RW_QKV; i++) {
          S.pub[C::RW_QKV * cw + i] = ya[i] * row_scale_of<WD>(sq[i]) * ia;
          S.pub[16 + C::RW_QKV * cw + i] = yb[i] * row_scale_of<WD>(sq[i]) * ib;
        }
      }
      publish_pair<W, false>(S, c.region, c.slots, LY.e1 + 16 * r, LY.b1 + 16 * r, 16, c.tick(f, l, 0), lane);
      if (cw == 2) {  // the second row's S2 input
        sleep_units(c.dl[Ws::kHopS2]);
        const bool ok = poll_cells<mb(512), false, kLO>(c.region, c.slots, LY.b1, 512, c.tick(f, l, 0), P.qkv,
                                                        c.ws, lane, c, 12u, f, l);
        if (!ok && lane == 0) P.bad = 1;
      }
      load_w<WD, C::RW_GU, C::CH, kLO, KEEP>(wg, sg, gg, (const int8_t*)Ly.gu_w, Ly.gu_s, gu_w0, C::RW_GU, H, lane);
    }
    // ---- S2: attention of both positions over positions 0 and 1
    wg_sync();
    if (S.flags[1] || P.bad) return false;
    {
      // (1) wave vw normalises and rotates vector vw (q0, q1, k, v) of both rows; workgroup 0 of the head
      // appends both K/V rows
      const int vw = cw & 3;
      const float b_cs = gload(c.d.rope + (size_t)(c.pos0 + 1) * SK_HD + lane);
      const float b_sn = gload(c.d.rope + (size_t)(c.pos0 + 1) * SK_HD + 64 + lane);
#pragma unroll
      for (int row = 0; row < 2; row++) {
        const float* src = row ? P.qkv : S.qkv;
        const float cs = row ? b_cs : a_cs, sn = row ? b_sn : a_sn;
        const float x0 = src[vw * SK_HD + lane], x1 = src[vw * SK_HD + 64 + lane];
        const float inv = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / SK_HD + eps);
        const float n0 = x0 * inv * a_n0, n1 = x1 * inv * a_n1;
        const float r0 = n0 * cs - n1 * sn, r1 = n1 * cs + n0 * sn;  // rotate-half RoPE
        if (cw < 2) {
          float* qd = row ? P.qs[cw] : S.qs[cw];
          qd[lane] = r0 * kInvSqrtHd;
          qd[lane + 64] = r1 * kInvSqrtHd;
        } else if (cw < 4) {
          const float y0 = bf2f(f2bf(cw == 2 ? r0 : x0)), y1 = bf2f(f2bf(cw == 2 ? r1 : x1));
          float* dst = cw == 2 ? (row ? P.kn : S.kn) : (row ? P.vn : S.vn);
          dst[lane] = y0;
          dst[lane + 64] = y1;
          if (r == 0) {
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(uniform(cw == 2 ? c.kh(Ly) : c.vh(Ly)));
            const uint32_t off = (uint32_t)((c.pos0 + row) * SK_HD + lane) * 2u;
            __builtin_amdgcn_raw_buffer_store_b16(f2bf(y0), rs, off, 0, kPolDev);
            __builtin_amdgcn_raw_buffer_store_b16(f2bf(y1), rs, off + 128u, 0, kPolDev);
          }
        }
      }
      wg_sync();  // paired barrier 1
      // (2) the second row's scores at positions 0 and 1: head p's q . k over the head's two waves
      {
        const float qb = P.qs[p][dd];
        const float s0 = wave_sum(qb * S.kn[dd]), s1 = wave_sum(qb * P.kn[dd]);
        if (lane == 0) { P.red[2 * cw] = s0; P.red[2 * cw + 1] = s1; }
      }
      wg_sync();  // paired barrier 2
      {
        // waves 2p and 2p + 1 hold head p; the first row's output is v at position 0 (weight 1)
        const float s0 = P.red[4 * p] + P.red[4 * p + 2], s1 = P.red[4 * p + 1] + P.red[4 * p + 3];
        const float m = fmaxf(s0, s1), e0 = expf(s0 - m), e1 = expf(s1 - m);
        const float oa = S.vn[dd], ob = (e0 * S.vn[dd] + e1 * P.vn[dd]) / (e0 + e1);
        // this workgroup's slice of the S4 inputs (q head 2x + r/16, dims 8 (r % 16) .. + 8), as the whole-cache
        // attention writes it
        if (p == (r >> 4) && (dd >> 3) == (r & 15)) {
          put_all(c.region, LY.e3 + (2 * x + p) * SK_HD + dd, oa, c.tick(f, l, 2));
          put_all(c.region, LY.b3 + (2 * x + p) * SK_HD + dd, ob, c.tick(f, l, 2));
        }
      }
      if (cw < kQ / 1024) {  // the second row's S4 input, 1024 cells per wave (staged from element 1024 cw)
        sleep_units(c.dl[Ws::kHopS4]);
        const bool ok = poll_cells<mb(1024), true, kLO>(c.region, c.slots, LY.b3 + 1024u * cw, 1024, c.tick(f, l, 2),
                                                        P.xs[1] + xsw(1024 * cw), c.ws, lane, c, 14u, f, l);
        if (!ok && lane == 0) P.bad = 1;
      }
      load_attn_vec(Ln);
    }
    // ---- S4: o rows of both positions, added to their residuals
    wg_sync();
    if (S.flags[2] || P.bad) return false;
    {
      float ya[C::RW_O], yb[C::RW_O];
      dot2_w<WD, C::RW_O, C::CQ>(wo, go, S.xs[1], P.xs[1], lane, ya, yb);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < C::RW_O; i++)
          if (i < o_wn) {
            S.pub[C::RW_O * cw + i] = S.hin[o_w0 + i] + ya[i] * row_scale_of<WD>(so[i]);
            S.pub[C::R_O + C::RW_O * cw + i] = P.hin[o_w0 + i] + yb[i] * row_scale_of<WD>(so[i]);
          }
      }
      publish_pair<W, true>(S, c.region, c.slots, LY.e4 + C::R_O * g, LY.b4 + C::R_O * g, C::R_O, c.tick(f, l, 3), lane);
      if (cw == 3) {  // the second row's S5 input: its residual after o, times the post-attention norm
        sleep_units(c.dl[Ws::kHopS5]);
        u32x4 q[kNP];
        float2 v[kNP];
        const bool ok = poll_regs<kNP, kLO>(c.region, c.slots, LY.b4, c.tick(f, l, 3), q, c.ws, lane, c, 15u, f, l);
        if (!ok && lane == 0) P.bad = 1;
        cells_to_pairs<kNP>(q, v);
        stage_b(v, Ly.post_norm, P.hmid);
      }
      load_w<WD, C::RW_D, C::CI, kLO, KEEP>(wd, sd, gd, (const int8_t*)Ly.down_w, Ly.down_s, d_w0, d_wn, I, lane);
    }
    // ---- S5: gate/up rows of both positions, SwiGLU
    wg_sync();
    if (S.flags[3] || P.bad) return false;
    {
      float ya[C::RW_GU], yb[C::RW_GU];
      dot2_w<WD, C::RW_GU, C::CH>(wg, gg, S.xs[0], P.xs[0], lane, ya, yb);
      const float ia = S.inv, ib = P.inv;
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < C::RW_GU; i += 2) {
          S.pub[(C::RW_GU * cw + i) / 2] = silu_mul(ya[i] * row_scale_of<WD>(sg[i]) * ia, ya[i + 1] * row_scale_of<WD>(sg[i + 1]) * ia);
          S.pub[C::R_GU / 2 + (C::RW_GU * cw + i) / 2] =
              silu_mul(yb[i] * row_scale_of<WD>(sg[i]) * ib, yb[i + 1] * row_scale_of<WD>(sg[i + 1]) * ib);
        }
      }
      publish_pair<W, true>(S, c.region, c.slots, LY.e5 + C::R_GU / 2 * g, LY.b5 + C::R_GU / 2 * g, C::R_GU / 2,
                            c.tick(f, l, 4), lane);
      if (cw < I / 1024) {  // the second row's S6 input, 1024 cells per wave
        sleep_units(c.dl[Ws::kHopS6]);
        const bool ok = poll_cells<mb(1024), true, kLO>(c.region, c.slots, LY.b5 + 1024u * cw, 1024, c.tick(f, l, 4),
                                                        P.xs[1] + xsw(1024 * cw), c.ws, lane, c, 16u, f, l);
        if (!ok && lane == 0) P.bad = 1;
      }
      load_w<WD, C::RW_QKV, C::CH, kLO, KEEP>(wq, sq, gq, (const int8_t*)Ln.qkv_w, Ln.qkv_s, q_w0, C::RW_QKV, H, lane);
    }
    // ---- S6: down rows of both positions, added to their residuals after o
    wg_sync();
    if (S.flags[4] || P.bad) return false;
    {
      float ya[C::RW_D], yb[C::RW_D];
      dot2_w<WD, C::RW_D, C::CI>(wd, gd, S.xs[1], P.xs[1], lane, ya, yb);
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < C::RW_D; i++) {
          if (i < d_wn) {
            const float hb = P.hmid[d_w0 + i] + yb[i] * row_scale_of<WD>(sd[i]);
            S.pub[C::RW_D * cw + i] = S.hmid[d_w0 + i] + ya[i] * row_scale_of<WD>(sd[i]);
            S.pub[C::R_D + C::RW_D * cw + i] = hb;
            if (c.d.layer_out && c.n_frames == 2) gstore(c.d.layer_out + (size_t)l * H + d_w0 + i, hb);
          }
        }
      }
      publish_pair<W, true>(S, c.region, c.slots, LY.e6 + C::R_D * g, LY.b6 + C::R_D * g, C::R_D, c.tick(f, l, 5), lane);
      load_w<WD, C::RW_O, C::CQ, kLO, KEEP>(wo, so, go, (const int8_t*)Ln.o_w, Ln.o_s, o_w0, o_wn, kQ, lane);
    }
  }
  return true;
}

template <int H, int I, int W, int V, bool CP, bool SMP, int WD, bool KEEP, bool F16 = false>
__device__ void run_compute(const Ctx& c, Lds<H, I, W, V, CP>& S, int cw, int tid, int lane) {
  using C = CfgW<H, I, W, V, CP, WD>;
  constexpr bool kLO = LaneOffsetPolls<H>::value;
  const Layout LY(H, I);
  const float eps = c.d.eps;
  const int ag = lane >> 4, asl = lane & 15;
  const int x = (int)c.x, r = c.r, g = c.g;
  // S1 rows: 512 rows of head x (q of heads 2x, 2x+1, then k and v of head x), 16 per workgroup
  int qkv_row0;
  if (r < 16) qkv_row0 = 256 * x + 16 * r;
  else if (r < 24) qkv_row0 = kQ + 128 * x + 16 * (r - 16);
  else qkv_row0 = kQ + kNKV * 128 + 128 * x + 16 * (r - 24);
  const int q_w0 = qkv_row0 + C::RW_QKV * cw;
  // With more waves than rows (RW * W > R) a wave with no rows of its own loads the workgroup's last row (in range,
  // values unused; load_rows repeats row0 for rows past nvalid) instead of one past the workgroup's rows, which is
  // past the matrix for the last workgroup.
  constexpr bool kClO = C::RW_O * W > C::R_O, kClD = C::RW_D * W > C::R_D, kClH = C::RW_HEAD * W > C::kHeadRows;
  const int o_w0 = C::R_O * g + (kClO ? min(C::RW_O * cw, C::R_O - 1) : C::RW_O * cw), o_wn = max(0, min(C::RW_O, C::R_O - C::RW_O * cw));
  const int gu_w0 = C::R_GU * g + C::RW_GU * cw;
  const int d_w0 = C::R_D * g + (kClD ? min(C::RW_D * cw, C::R_D - 1) : C::RW_D * cw), d_wn = max(0, min(C::RW_D, C::R_D - C::RW_D * cw));
  const int h_w0 = C::kHeadRows * g + (kClH ? min(C::RW_HEAD * cw, C::kHeadRows - 1) : C::RW_HEAD * cw),
            h_wn = max(0, min(C::RW_HEAD, C::kHeadRows - C::RW_HEAD * cw));

  // code predictor: lane f holds position f's head weights and scales (read once, not per position)
  const uint64_t head_w_l = (CP && lane < c.d.max_len) ? (uint64_t)gload(c.cp.head_w + lane) : 0;
  const uint64_t head_s_l = (CP && lane < c.d.max_len) ? (uint64_t)gload(c.cp.head_s + lane) : 0;
  uint4 wq[C::RW_QKV][C::CH], wo[C::RW_O][C::CQ], wg[C::RW_GU][C::CH], wd[C::RW_D][C::CI];
  uint16_t sq[C::RW_QKV], so[C::RW_O], sg[C::RW_GU], sd[C::RW_D];  // raw bf16 row scales
  constexpr bool G32 = WD == SK_WD_I8G32;  // i8g32: raw fp16 group scales, one per row and chunk
  constexpr bool kSplitGu = C::kSpread && SplitGateUp<H, I>::value && C::RW_GU % 2 == 0;
  constexpr int kGuH = C::RW_GU / 2;
  uint16_t gq[G32 ? C::RW_QKV : 1][G32 ? C::CH : 1], go[G32 ? C::RW_O : 1][G32 ? C::CQ : 1];
  uint16_t gg[G32 ? C::RW_GU : 1][G32 ? C::CH : 1], gd[G32 ? C::RW_D : 1][G32 ? C::CI : 1];
  uint4 kr[C::KVL], vr[C::KVL];
  // A projected code predictor (CpProjIn): each wave holds one row of the projection for the whole launch (rows
  // 4 g .. 4 g + 3 of the workgroup; PK = 2048: 2 chunks per lane for int8, 4 for bf16) and its bias
  constexpr int PK = CP ? CpProjIn<H, I>::value : 0;
  constexpr int CPJ = PK > 0 ? PK / 1024 * C::WB : 1;
  static_assert(PK == 0 || (H / kWG == W && PK % 1024 == 0), "one projection row per compute wave");
  uint4 wpj[1][CPJ];
  uint16_t spj[1];
  uint16_t gpj[1][G32 && PK > 0 ? CPJ : 1];
  float pbias = 0.f;
  const int prow = (H / kWG) * g + cw;
  auto load_proj = [&]() {
    if constexpr (PK > 0) load_w<WD, 1, CPJ, kLO>(wpj, spj, gpj, (const int8_t*)c.cp.proj_w, c.cp.proj_s, prow, 1, PK, lane);
  };
  // F16 (a code-predictor launch of at most 16 positions): wave 0 computes this workgroup's attention slice alone,
  // from K / V loaded in load_kv16's layout
  constexpr bool kF16 = CP && F16;
  uint4 kf[kF16 ? 4 : 1];
  uint32_t vf = 0;
  const int sl_p = r >> 4, sl_d0 = 8 * (r & 15);  // the slice: q head 2x + sl_p, dims sl_d0 .. sl_d0 + 7
  // RoPE row (cos, sin of pair `lane`) and the norm weights of dims lane, lane + 64 for this wave's vector in
  // the next attention (q norm for waves 0, 1, k norm for wave 2; loaded by every compute wave: no select on
  // loaded values, only on the address)
  float a_cs = 0.f, a_sn = 0.f, a_n0 = 0.f, a_n1 = 0.f;
  auto load_attn_vec = [&](const sk_layer_desc& Lx, int posx) {
    const float* nw = (cw & 3) == 2 ? Lx.kn : Lx.qn;
    a_cs = gload(c.d.rope + (size_t)posx * SK_HD + lane);
    a_sn = gload(c.d.rope + (size_t)posx * SK_HD + 64 + lane);
    a_n0 = gload(nw + lane);
    a_n1 = gload(nw + 64 + lane);
  };
  const int f0 = CP && c.cp.pair ? 1 : 0;  // the frame loop's first frame: 1 after the paired pass (its own launch)
  // the first frame with layers: 0, or 2 after a paired pass (position 2 < max_len when there is a frame 2)
  const int p0 = c.pos0 + (f0 && c.n_frames > 2 ? 2 : 0);
  {
    const sk_layer_desc& L0 = S.desc[0];
    if constexpr (PK > 0) {
      load_w<WD, 1, CPJ, kLO>(wpj, spj, gpj, (const int8_t*)c.cp.proj_w, c.cp.proj_s, prow, 1, PK, lane);
      if (c.cp.proj_b) pbias = gload(c.cp.proj_b + prow);
    }
    load_w<WD, C::RW_QKV, C::CH, kLO, KEEP>(wq, sq, gq, (const int8_t*)L0.qkv_w, L0.qkv_s, q_w0, C::RW_QKV, H, lane);
    if constexpr (kF16) load_kv16(kf, vf, c.kh(L0), c.vh(L0), p0, sl_d0, lane);
    else load_kv<W, C::KVL>(kr, vr, c.kh(L0), c.vh(L0), make_chunk<CP>(p0, r, C::whole(p0)), cw, ag, asl);
    load_attn_vec(L0, p0);
    if constexpr (!C::kLate) {
      load_w<WD, C::RW_O, C::CQ, kLO, KEEP>(wo, so, go, (const int8_t*)L0.o_w, L0.o_s, o_w0, o_wn, kQ, lane);
      load_w<WD, C::RW_GU, C::CH, kLO, KEEP>(wg, sg, gg, (const int8_t*)L0.gu_w, L0.gu_s, gu_w0, C::RW_GU, H, lane);
      load_w<WD, C::RW_D, C::CI, kLO, KEEP>(wd, sd, gd, (const int8_t*)L0.down_w, L0.down_s, d_w0, d_wn, I, lane);
    }
  }
  const bool block_eos0 = c.d.talker_processor && c.d.ngen;
  const int64_t ngen0 = c.d.ngen ? gload(c.d.ngen) : 0;
  // Wait once for the first layer's loads. The compiler places one static wait count per use; without this it
  // would have to allow for the prologue's own load order on every layer, and waits would come out shallow.
  __builtin_amdgcn_s_waitcnt(0);
  for (int f = f0; f < c.n_frames; f++) {
    const int pos = c.pos0 + f;
    const auto ck = make_chunk<CP>(pos, r, C::whole(pos));
    const bool pr = CP && c.cp.pair;
    // ---- S0 (a projected code predictor): this wave's projection row, plus the bias, before the position's
    // layers. The row was loaded after the previous position's head (its registers are the head's), or in the
    // prologue for position 0; outside the layer loop it is live only from that load to this dot.
    if constexpr (PK > 0) {
      wg_sync();  // the projection's input is staged
      float y[1];
      dot_w<WD, 1, CPJ>(wpj, gpj, S.xs[0], lane, y);
      if (lane == 0) S.pub[cw] = y[0] * row_scale_of<WD>(spj[0]) + pbias;
      publish<W, true, C::kSingle>(S, c.region, c.slots, LY.pj + (uint32_t)(H / kWG) * g, H / kWG, c.tick(f, 0, 6), lane);
    }
    for (int l = 0; l < (pr && f == 1 ? 0 : c.L); l++) {
      const sk_layer_desc& Ly = S.desc[l];
      const bool last_layer = l == c.L - 1;
      const sk_layer_desc& Ln = S.desc[last_layer ? 0 : l + 1];
      // The next layer's weights and K/V are prefetched unconditionally (after the last layer of the last frame
      // that reloads layer 0, unused): a prefetch under a condition makes the compiler assume it may not have
      // been issued, and then every later wait for older loads also waits for the younger ones.
      const int npos = (last_layer && f + 1 < c.n_frames) ? pos + 1 : pos;  // always < max_len
      // ---- S1: qkv rows -----------------------------------------------------------------------------------
      wg_sync();
      if (S.flags[0]) return;
      if (tid == 0) c.tr(1, f, l, 0);
      {
        float y[C::RW_QKV];
        dot_w<WD, C::RW_QKV, C::CH>(wq, gq, S.xs[0], lane, y);
        if (tid == 0) c.tr(1, f, l, 8);
        const float inv = S.inv;
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < C::RW_QKV; i++) S.pub[C::RW_QKV * cw + i] = y[i] * row_scale_of<WD>(sq[i]) * inv;
        }
        publish<W, false>(S, c.region, c.slots, LY.e1 + 16 * r, 16, c.tick(f, l, 0), lane);
        if (tid == 0) c.tr(1, f, l, 1);
        if constexpr (!C::kLate) load_w<WD, C::RW_QKV, C::CH, kLO, KEEP>(wq, sq, gq, (const int8_t*)Ln.qkv_w, Ln.qkv_s, q_w0, C::RW_QKV, H, lane);
        // With gate/up split over two exchanges (SplitGateUp) the o rows go out here, before the attention, rather
        // than after it with the first gate/up half: the merge's poll then does not queue behind them (1.7B: 22.96
        // against 23.25 us per layer; moving the first gate/up half here too measured 23.8)
        if constexpr (C::kLate && kSplitGu) load_w<WD, C::RW_O, C::CQ, kLO, KEEP>(wo, so, go, (const int8_t*)Ly.o_w, Ly.o_s, o_w0, o_wn, kQ, lane);
      }
      // ---- S2: attention over this workgroup's chunk ----------------------------------------------------
      wg_sync();
      if (S.flags[1]) return;
      if (tid == 0) c.tr(1, f, l, 2);
      {
        const bool has_pos = ck.has_pos();
        // (1) one wave per vector, two dims per lane (d and d + 64, the RoPE pair): wave 0 q of head 2x, wave 1 q
        // of head 2x + 1, wave 2 k, wave 3 v. RMSNorm over the head is a wave reduction, RoPE stays in the lane.
        {
          const int vw = cw & 3;
          const float x0 = S.qkv[vw * SK_HD + lane], x1 = S.qkv[vw * SK_HD + 64 + lane];
          const float inv = rsqrtf(wave_sum(x0 * x0 + x1 * x1) / SK_HD + eps);
          const float n0 = x0 * inv * a_n0, n1 = x1 * inv * a_n1;
          const float r0 = n0 * a_cs - n1 * a_sn, r1 = n1 * a_cs + n0 * a_sn;  // rotate-half RoPE
          if (cw < 2) {
            S.qs[cw][lane] = r0 * kInvSqrtHd;
            S.qs[cw][lane + 64] = r1 * kInvSqrtHd;
          } else if (cw < 4) {
            // k (normalised, rotated) or v (as is), rounded to the cache's bf16; the owner of pos appends them
            // (device-coherent: later frames read them from other workgroups)
            const float y0 = bf2f(f2bf(cw == 2 ? r0 : x0)), y1 = bf2f(f2bf(cw == 2 ? r1 : x1));
            float* dst = cw == 2 ? S.kn : S.vn;
            dst[lane] = y0;
            dst[lane + 64] = y1;
            if (has_pos) {
              const __amdgpu_buffer_rsrc_t rs = make_rsrc(uniform(cw == 2 ? c.kh(Ly) : c.vh(Ly)));
              if constexpr (kLO) {
                const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)pos * SK_HD * 2u);
                __builtin_amdgcn_raw_buffer_store_b16(f2bf(y0), rs, (uint32_t)lane * 2u, so, kPolDev);
                __builtin_amdgcn_raw_buffer_store_b16(f2bf(y1), rs, (uint32_t)lane * 2u + 128u, so, kPolDev);
              } else {
                const uint32_t off = (uint32_t)(pos * SK_HD + lane) * 2u;
                __builtin_amdgcn_raw_buffer_store_b16(f2bf(y0), rs, off, 0, kPolDev);
                __builtin_amdgcn_raw_buffer_store_b16(f2bf(y1), rs, off + 128u, 0, kPolDev);
              }
            }
          }
        }
        wg_sync();  // attention barrier 1
        if constexpr (kF16) {
          // (2') wave 0: this workgroup's slice over the whole cache (<= 16 positions), no further barrier. Lane
          // 16 qq + j: q . k_j over dims 32 qq .. + 31, summed over the four quarters; softmax over j within
          // each row; the slice's dims 2 qq, 2 qq + 1 summed over j within the row.
          if (cw == 0) {
            const int j = lane & 15, qq = lane >> 4;
            float k32[32];
            if (j == pos) {
#pragma unroll
              for (int e = 0; e < 32; e++) k32[e] = S.kn[32 * qq + e];
            } else {
#pragma unroll
              for (int e = 0; e < 4; e++) unpack8(kf[e], k32 + 8 * e);
            }
            float sc = 0.f;
#pragma unroll
            for (int e = 0; e < 32; e++) sc = __builtin_fmaf(S.qs[sl_p][32 * qq + e], k32[e], sc);
            sc += __shfl_xor(sc, 16);
            sc += __shfl_xor(sc, 32);
            const float sv = j <= pos ? sc : -INFINITY;
            const float mx = row16_max(sv);
            const float ew = j <= pos ? expf(sv - mx) : 0.f;
            const float lw = row16_sum(ew);
            const float v0 = j == pos ? S.vn[sl_d0 + 2 * qq] : bf2f(vf & 0xffffu);
            const float v1 = j == pos ? S.vn[sl_d0 + 2 * qq + 1] : bf2f(vf >> 16);
            const float o0 = row16_sum(ew * v0), o1 = row16_sum(ew * v1);
            // every lane of a row holds the row's sums: lane j < 8 stores copy j
            if (j < kXcd) {
              const uint32_t e = c.tick(f, l, 2);
              const u32x4 y = {__float_as_uint(lw > 0.f ? o0 / lw : 0.f), e, __float_as_uint(lw > 0.f ? o1 / lw : 0.f), e};
              __builtin_amdgcn_raw_buffer_store_b128(y, make_rsrc(c.region),
                                                     ((uint32_t)j << 12) +
                                                         cell_off(LY.e3 + (2 * x + sl_p) * SK_HD + sl_d0 + 2 * qq),
                                                     0, kPolDev);
            }
          }
        } else {
        // P V by dimension slice (load_kv's V layout), published straight from the registers (no third barrier); ov
        // is this lane's output dim, m0v .. l1v the softmax statistics it is published with
        float ov = 0.f;
        float m0v = -INFINITY, m1v = -INFINITY, l0v = 0.f, l1v = 0.f;
        if (ck.n > 0) {
          // (2) scores of this chunk's positions (kr from the prefetch; the new position from LDS)
          {
            float q0[8], q1[8];
#pragma unroll
            for (int e = 0; e < 8; e++) { q0[e] = S.qs[0][8 * asl + e]; q1[e] = S.qs[1][8 * asl + e]; }
#pragma unroll
            for (int i = 0; i < C::KVL; i++) {
              const int jj = 4 * W * i + 4 * cw + ag;
              float k8[8];
              if (jj < ck.n && ck.t0 + jj == pos) {
#pragma unroll
                for (int e = 0; e < 8; e++) k8[e] = S.kn[8 * asl + e];
              } else {
                unpack8(kr[i], k8);
              }
              float s0 = 0.f, s1 = 0.f;
#pragma unroll
              for (int e = 0; e < 8; e++) { s0 = __builtin_fmaf(q0[e], k8[e], s0); s1 = __builtin_fmaf(q1[e], k8[e], s1); }
              s0 = row16_sum(s0);
              s1 = row16_sum(s1);
              if (asl == 0 && jj < ck.n) { S.sc[0][jj] = s0; S.sc[1][jj] = s1; }
            }
          }
          wg_sync();  // 2
          // (3) softmax statistics, computed by every wave from the chunk's scores (at most 64 per head)
          static_assert(C::kMaxChunk <= 64, "one score per lane");
          const int jl = min(lane, C::kMaxChunk - 1);
          const float s0l = lane < ck.n ? S.sc[0][jl] : -INFINITY, s1l = lane < ck.n ? S.sc[1][jl] : -INFINITY;
          const float m0 = wave_max(s0l), m1 = wave_max(s1l);
          const float l0 = wave_sum(lane < ck.n ? expf(s0l - m0) : 0.f), l1 = wave_sum(lane < ck.n ? expf(s1l - m1) : 0.f);
          {
            // (4') P V of this wave's 32 dims over every position of the chunk: lane (ag, asl) takes positions
            // asl + 16 i, dims 32 cw + 8 ag .. + 7; the row's sums then land one per lane, lane asl holding dim
            // 32 cw + 8 ag + (asl % 8) of head asl / 8
            float a[16];
#pragma unroll
            for (int e = 0; e < 16; e++) a[e] = 0.f;
#pragma unroll
            for (int i = 0; i < C::KVL; i++) {
              const int jj = asl + 16 * i;
              if (jj < ck.n) {
                float v8[8];
                if (ck.t0 + jj == pos) {
#pragma unroll
                  for (int e = 0; e < 8; e++) v8[e] = S.vn[32 * cw + 8 * ag + e];
                } else {
                  unpack8(vr[i], v8);
                }
                const float e0 = expf(S.sc[0][jj] - m0), e1 = expf(S.sc[1][jj] - m1);
#pragma unroll
                for (int e = 0; e < 8; e++) { a[e] = __builtin_fmaf(e0, v8[e], a[e]); a[8 + e] = __builtin_fmaf(e1, v8[e], a[8 + e]); }
              }
            }
            ov = row16_reduce_scatter(a, lane);
            m0v = m0; m1v = m1; l0v = l0; l1v = l1;
          }
        }
        {
          const int ph = asl >> 3, dsl = 32 * cw + 8 * ag + (asl & 7);
          if (ck.whole) {
            // the whole cache in this workgroup: its slice of the S4 input (q head 2x + r/16, dims 8 (r % 16) ..
            // + 8), normalised, as the merge would write it
            const float lw = ph ? l1v : l0v;
            if (ph == (r >> 4) && (dsl >> 3) == (r & 15))
              put_all<C::kSingle>(c.region, LY.e3 + (2 * x + ph) * SK_HD + dsl, lw > 0.f ? ov / lw : 0.f, c.tick(f, l, 2));
          } else {
            // publish the partial (this XCD's copy): m0 l0 m1 l1 at e2m + 4 r, o0[128] o1[128] at e2o + 256 r
            const uint32_t pm = LY.e2m + 4u * (uint32_t)r, po = LY.e2o + 2u * SK_HD * (uint32_t)r;
            const uint32_t e = c.tick(f, l, 1);
            if constexpr (kLO) {
              if (cw == 0 && lane < 4)
                putl(c.region, c.slots, pm, (uint32_t)lane * 8u, lane == 0 ? m0v : lane == 1 ? l0v : lane == 2 ? m1v : l1v, e);
              putl(c.region, c.slots, po, (uint32_t)(ph * SK_HD + dsl) * 8u, ov, e);
            } else {
              if (cw == 0 && lane < 4) put(c.region, c.slots, pm + lane, lane == 0 ? m0v : lane == 1 ? l0v : lane == 2 ? m1v : l1v, e);
              put(c.region, c.slots, po + ph * SK_HD + dsl, ov, e);
            }
          }
        }
        }
        if (tid == 0) c.tr(1, f, l, 3);
        if constexpr (!C::kSpread) {
          if constexpr (kF16) load_kv16(kf, vf, c.kh(Ln), c.vh(Ln), npos, sl_d0, lane);
          else load_kv<W, C::KVL>(kr, vr, c.kh(Ln), c.vh(Ln), make_chunk<CP>(npos, r, C::whole(npos)), cw, ag, asl);
          load_attn_vec(Ln, npos);
        }
        if constexpr (C::kLate) {
          if constexpr (!kSplitGu) load_w<WD, C::RW_O, C::CQ, kLO, KEEP>(wo, so, go, (const int8_t*)Ly.o_w, Ly.o_s, o_w0, o_wn, kQ, lane);
          if constexpr (!C::kSpread) {
            load_w<WD, C::RW_GU, C::CH, kLO, KEEP>(wg, sg, gg, (const int8_t*)Ly.gu_w, Ly.gu_s, gu_w0, C::RW_GU, H, lane);
          } else if constexpr (kSplitGu) {  // the first half of the gate/up rows
            load_w<WD, kGuH, C::CH, kLO, KEEP>(*(uint4(*)[kGuH][C::CH]) & wg[0], *(uint16_t(*)[kGuH]) & sg[0],
                                               *(uint16_t(*)[G32 ? kGuH : 1][G32 ? C::CH : 1]) & gg[0],
                                               (const int8_t*)Ly.gu_w, Ly.gu_s, gu_w0, kGuH, H, lane);
          }
        }
      }
      // ---- S4: o projection rows, added to the layer's input residual ------------------------------------
      wg_sync();
      if (S.flags[2]) return;
      if (tid == 0) c.tr(1, f, l, 4);
      {
        float y[C::RW_O];
        if (tid == 0) c.tr_clk(1, f, l, 14);
        dot_w<WD, C::RW_O, C::CQ>(wo, go, S.xs[1], lane, y);
        if (tid == 0) c.tr(1, f, l, 9);
        if (tid == 0) c.tr_clk(1, f, l, 15);
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < C::RW_O; i++)
            if (i < o_wn) S.pub[C::RW_O * cw + i] = S.hin[o_w0 + i] + y[i] * row_scale_of<WD>(so[i]);
        }
        publish<W, true, C::kSingle>(S, c.region, c.slots, LY.e4 + C::R_O * g, C::R_O, c.tick(f, l, 3), lane);
        if (tid == 0) c.tr(1, f, l, 5);
        if constexpr (!C::kLate) load_w<WD, C::RW_O, C::CQ, kLO, KEEP>(wo, so, go, (const int8_t*)Ln.o_w, Ln.o_s, o_w0, o_wn, kQ, lane);
        if constexpr (C::kSpread && kSplitGu) {  // the second half of the gate/up rows
          load_w<WD, kGuH, C::CH, kLO, KEEP>(*(uint4(*)[kGuH][C::CH]) & wg[kGuH], *(uint16_t(*)[kGuH]) & sg[kGuH],
                                             *(uint16_t(*)[G32 ? kGuH : 1][G32 ? C::CH : 1]) & gg[G32 ? kGuH : 0],
                                             (const int8_t*)Ly.gu_w, Ly.gu_s, gu_w0 + kGuH, kGuH, H, lane);
        } else if constexpr (C::kSpread) {
          load_w<WD, C::RW_GU, C::CH, kLO, KEEP>(wg, sg, gg, (const int8_t*)Ly.gu_w, Ly.gu_s, gu_w0, C::RW_GU, H, lane);
        }
      }
      // ---- S5: gate/up rows with the RMSNorm scale, SwiGLU ----------------------------------------------
      wg_sync();
      if (S.flags[3]) return;
      if (tid == 0) c.tr(1, f, l, 12);
      {
        float y[C::RW_GU];
        dot_w<WD, C::RW_GU, C::CH>(wg, gg, S.xs[0], lane, y);
        if (tid == 0) c.tr(1, f, l, 10);
        const float inv = S.inv;
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < C::RW_GU; i += 2)
            S.pub[(C::RW_GU * cw + i) / 2] = silu_mul(y[i] * row_scale_of<WD>(sg[i]) * inv, y[i + 1] * row_scale_of<WD>(sg[i + 1]) * inv);
        }
        publish<W, true, C::kSingle>(S, c.region, c.slots, LY.e5 + C::R_GU / 2 * g, C::R_GU / 2, c.tick(f, l, 4), lane);
        if (tid == 0) c.tr(1, f, l, 6);
        if constexpr (C::kLate) {
          load_w<WD, C::RW_D, C::CI, kLO, KEEP>(wd, sd, gd, (const int8_t*)Ly.down_w, Ly.down_s, d_w0, d_wn, I, lane);
          if constexpr (!C::kSpread)
            load_w<WD, C::RW_QKV, C::CH, kLO, KEEP>(wq, sq, gq, (const int8_t*)Ln.qkv_w, Ln.qkv_s, q_w0, C::RW_QKV, H, lane);
        } else {
          load_w<WD, C::RW_GU, C::CH, kLO, KEEP>(wg, sg, gg, (const int8_t*)Ln.gu_w, Ln.gu_s, gu_w0, C::RW_GU, H, lane);
        }
      }
      // ---- S6: down rows, added to the residual after o --------------------------------------------------
      wg_sync();
      if (S.flags[4]) return;
      if (tid == 0) c.tr(1, f, l, 13);
      {
        float y[C::RW_D];
        dot_w<WD, C::RW_D, C::CI>(wd, gd, S.xs[1], lane, y);
        if (tid == 0) c.tr(1, f, l, 11);
        if (lane == 0) {
#pragma unroll
          for (int i = 0; i < C::RW_D; i++) {
            if (i < d_wn) {
              const float hv = S.hmid[d_w0 + i] + y[i] * row_scale_of<WD>(sd[i]);
              S.pub[C::RW_D * cw + i] = hv;
              if (c.d.layer_out && f == c.n_frames - 1) gstore(c.d.layer_out + (size_t)l * H + d_w0 + i, hv);
            }
          }
        }
        publish<W, true, C::kSingle>(S, c.region, c.slots, LY.e6 + C::R_D * g, C::R_D, c.tick(f, l, 5), lane);
        if (tid == 0) c.tr(1, f, l, 7);
        if constexpr (!C::kLate) load_w<WD, C::RW_D, C::CI, kLO, KEEP>(wd, sd, gd, (const int8_t*)Ln.down_w, Ln.down_s, d_w0, d_wn, I, lane);
        if constexpr (C::kSpread) {
          load_w<WD, C::RW_QKV, C::CH, kLO, KEEP>(wq, sq, gq, (const int8_t*)Ln.qkv_w, Ln.qkv_s, q_w0, C::RW_QKV, H, lane);
          if constexpr (kF16) load_kv16(kf, vf, c.kh(Ln), c.vh(Ln), npos, sl_d0, lane);
          else load_kv<W, C::KVL>(kr, vr, c.kh(Ln), c.vh(Ln), make_chunk<CP>(npos, r, C::whole(npos)), cw, ag, asl);
          load_attn_vec(Ln, npos);
        }
      }
    }
    if (CP && f == 0) {  // the code predictor's position 0 has no head
      __builtin_amdgcn_s_waitcnt(0);  // same drain as after a head (see below)
      load_proj();  // the next position's projection row
      continue;
    }
    // ---- head rows (loaded now; the final residual is a full layer away), processor, local argmax ----------
    uint4 wh[C::RW_HEAD][C::CH];
    uint16_t sh[C::RW_HEAD];
    uint16_t gh[G32 ? C::RW_HEAD : 1][G32 ? C::CH : 1];
    const int8_t* hw = CP ? (const int8_t*)lane_u64(head_w_l, f) : (const int8_t*)c.d.head_w;
    const uint16_t* hsc = CP ? (const uint16_t*)lane_u64(head_s_l, f) : c.d.head_s;
    load_w<WD, C::RW_HEAD, C::CH, kLO>(wh, sh, gh, hw, hsc, h_w0, h_wn, H, lane);
    wg_sync();
    if (S.flags[5]) return;
    {
      float y[C::RW_HEAD];
      dot_w<WD, C::RW_HEAD, C::CH>(wh, gh, S.xs[0], lane, y);
      const float inv = S.inv;
      const bool block_eos = block_eos0 && (ngen0 + f) < c.d.min_new;
      uint64_t best = 0;
      // The rows' values (seen-byte masks and offsets) are recomputed each frame: hoisted out of the frame loop they
      // stayed live across it and spilled (spilled VGPRs 0.6B 1 -> 0, 1.7B 5 -> 2, 1.7B i8g32 15 -> 3), and in the
      // sampling kernels their reloads sat in this serial lane-0 loop (0.5 us per frame)
      int hr0 = h_w0;
      __asm__ volatile("" : "+v"(hr0));
      if (lane == 0) {
#pragma unroll
        for (int i = 0; i < C::RW_HEAD; i++) {
          if (i >= h_wn) break;
          const int row = hr0 + i;
          float v = y[i] * row_scale_of<WD>(sh[i]) * inv;
          if (c.d.logits && f == c.n_frames - 1) gstore(c.d.logits + row, v);
          if (c.d.talker_processor) {
            if (c.d.seen && ((ld_u32_dev(uniform(c.d.seen), (uint32_t)row & ~3u) >> (8 * (row & 3))) & 0xffu))
              v = v < 0.f ? v * c.d.rep_pen : v / c.d.rep_pen;
            if (c.d.suppress && gload(c.d.suppress + row)) v = -INFINITY;
            if (block_eos && row == c.d.eos) v = -INFINITY;
          }
          if constexpr (SMP) S.hv[row - C::kHeadRows * g] = v * c.d.inv_temp;
          else if (v == v) { const uint64_t k = pick_key(v, row); best = k > best ? k : best; }
        }
        S.cand[cw] = best;
      }
    }
    load_proj();  // the next position's projection row, in flight during the pick (the head's registers are free)
    wg_sync();  // candidates ready for the control wave
    if constexpr (SMP)
      pick_compute<V, W, C::kSingle>(lds_addr((char*)&S + kPickCopy<H, I, W, V, CP>), lds_addr(S.xs[0]), lds_addr(S.xs[1]),
                         lds_addr((char*)&S + kPickShared<H, I, W, V, CP>), c.region, c.slots, c.ws, LY.e8, c.tick(f, c.L, 1),
                         c.cnt0 + (uint64_t)(CP ? f - 1 : f), c.seed, c.d.top_k, c.dl[Ws::kHopPick], f, c.L, c.g,
                         cw, lane, cw == 0 ? c.tslot(1, f, c.L, 0) : nullptr);
    wg_sync();  // pick done
    if (S.flags[6]) return;
    // The head dot already waited for the youngest loads; draining here keeps the next frame's first layer from
    // inheriting a shallow wait count from this path.
    __builtin_amdgcn_s_waitcnt(0);
  }
}

// SMP: sampled picks (do_sample != 0). The greedy instantiation carries none of the sampling code, whose call and
// registers would otherwise weigh on the control loop of every greedy frame.
// PAIRK: the code predictor's paired pass alone (positions 0 and 1, no head), launched before the frames of a
// cp.pair launch (which then start at frame 1's head): a kernel of its own, so that its registers do not add to
// the frame loop's (inlined into the same kernel, the pass made the loop's values spill).
template <int H, int I, int W, int V, bool CP, bool SMP, int WD, bool KEEP, bool PAIRK = false, bool F16 = false>
__global__ __launch_bounds__((W + 1) * 64) void k_frames(sk_talker_desc d, CpArgs cp, int n_frames) {
  extern __shared__ char smem_raw[];
  Lds<H, I, W, V, CP>& S = *(Lds<H, I, W, V, CP>*)smem_raw;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  void* ws = d.workspace;
  // ---- placement: XCD from hardware, dense rank from an arrival counter ------------------------------------
  __shared__ int s_rank;
  __shared__ uint32_t s_base, s_dl[2], s_trace, s_place[kQuarters];
  __shared__ int64_t s_pos0;
  const uint32_t x = xcc_id();
  // Every load of the prologue goes out before the first barrier, so the launch pays one memory round trip for
  // them instead of one per step: the layer descriptors (into LDS), the launch checks' inputs, the placement
  // census, the epoch base, the poll delays and the trace flag.
  for (int i = tid; i < d.n_layers * (int)(sizeof(sk_layer_desc) / 8); i += blockDim.x)
    ((uint64_t*)S.desc)[i] = gload((const uint64_t*)d.layers + i);
  if (wave == 0) {
    // the loads of the launch checks are issued together: lane g < in_groups reads talker_in code g (a serial loop
    // over the groups took one memory round trip per group before any workgroup could start)
    const int64_t cg = (!CP && lane < d.in_groups) ? gload(d.in_codes + lane) : 0;
    const int64_t pos0 = d.pos ? gload(d.pos) : 0, tok0 = gload(d.id0);
    const bool bad_code = __any(!CP && lane < d.in_groups && (cg < 0 || cg >= (lane == 0 ? d.vocab : d.in_rows)));
    if (lane == 0) {
    const uint32_t launch = ld_u32_dev(ws, Ws::kLaunch);
    const uint32_t old = __hip_atomic_fetch_add((uint32_t*)((char*)ws + Ws::kCensus + 4 * (x & 7)), 1u,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    int r = (int)(old - launch * kPerXcd);
    if (x >= kXcd || r < 0 || r >= kPerXcd) {
      st_u32_dev(ws, Ws::kErr, 2u);
      r = -1;
    }
    // every position this launch writes must lie inside the cache, and the start token inside the vocabulary.
    // A refused launch leaves the launch count behind the census; the host's reset (the whole workspace zeroed)
    // brings them back together.
    // talker_in codes: code 0 in the talker vocabulary, the rest in in_rows
    const bool bad = pos0 < 0 || pos0 + n_frames > d.max_len || tok0 < 0 || tok0 >= (CP ? cp.emb0_rows : d.vocab) || bad_code;
    if (bad) {
      st_u32_dev(ws, Ws::kErr, 5u);
      r = -1;
    }
    s_rank = r;
    s_base = ld_u32_dev(ws, Ws::kTick);
    s_dl[0] = ld_u32_dev(ws, Ws::kPollDelay);
    s_dl[1] = ld_u32_dev(ws, Ws::kPollDelay + 4);
    s_trace = ld_u32_dev(ws, Ws::kTraceOn);
    for (int q = 0; q < kQuarters; q++) s_place[q] = ld_u32_dev(ws, Ws::kPlace + 4 * q);
    s_pos0 = pos0;
    for (int i = 0; i < 8; i++) S.flags[i] = 0;
    S.pubcnt = 0;
    S.pubseq = 0;
    if constexpr (SMP) ((PickShared*)((char*)&S + kPickShared<H, I, W, V, CP>))->bad = 0u;
    }
  }
  __syncthreads();
  const int r = s_rank;
  if (r < 0) return;
  Ctx c;
  c.d = d;
  c.cp = cp;
  c.ws = ws;
  {
    // this XCD's page slot in each quarter of the region: the placement sk_frames_place measured where a quarter's
    // word carries one (bit 31) whose eight slots are distinct, else page x
    uint32_t slots = 0;
#pragma unroll
    for (int q = 0; q < kQuarters; q++) {
      const uint32_t w = __builtin_amdgcn_readfirstlane(s_place[q]);  // uniform: page offsets in scalar registers
      uint32_t used = 0;
#pragma unroll
      for (uint32_t i = 0; i < kXcd; i++) used |= 1u << ((w >> (3u * i)) & 7u);
      const uint32_t sl = ((w >> 31) && used == 0xffu) ? (w >> (3u * x)) & 7u : x;
      slots |= sl << (3 * q);
    }
    c.slots = slots;
    c.region = cell_region(ws);
  }
  c.x = x;
  c.r = r;
  c.g = (int)x * kPerXcd + r;
  c.tpf = (uint32_t)d.n_layers * 8u + 8u;
  // after a paired pass the frames' epochs continue from that launch's (frame 0 is the pass's)
  c.base = s_base - (CP && !PAIRK && cp.pair ? c.tpf : 0u);
  c.pos0 = (int)s_pos0;
  // read before this workgroup publishes anything: workgroup 0 advances the counter once every pick is done
  c.seed = SMP ? gload(d.seed) : 0;
  c.cnt0 = SMP ? gload(d.counter) : 0;
  c.n_frames = n_frames;
  c.L = d.n_layers;
  {
    // default start delays per exchange, overridable through the workspace: tuned by coordinate descent (a sweep of
    // 0-100 units per hop, then steps of 4 and 8) with the cells placed by sk_frames_place, on the 0.6B talker
    // (i8row; i8g32 keeps its set), on the 1.7B talker for the spread prefetch (i8row, and sets of its own for the
    // single-copy i8g32 and bf16 kernels), on the bf16 0.6B talker (spread prefetch at hidden 1024) and on the code
    // predictor (paired, and projected; sets of their own for bf16 weights). The merge poll (hop 2) starts after the
    // second attention barrier, before the compute waves' P V; a poll that starts before the partials are there
    // costs a whole extra round trip, so hop 2 keeps a margin over the measured edge. A second descent in steps of
    // 1-4 units followed. Per frame after tuning: 0.6B 354 us, 1.7B 633 / 675 / 967 (i8row / i8g32 / bf16), bf16
    // 0.6B 470, code predictor 846 (paired) and 911 (projected), bf16 957 and 1061.
    constexpr uint8_t kDefault[Ws::kHops] = {19, 20, 50, 20, 16, 31, 28, 13};
    constexpr uint8_t kDefaultSpread[Ws::kHops] = {38, 18, 74, 22, 50, 56, 46, 16};
    constexpr uint8_t kDefaultSpread17G32[Ws::kHops] = {57, 19, 64, 39, 35, 64, 12, 42};
    constexpr uint8_t kDefaultSpread06[Ws::kHops] = {34, 6, 60, 26, 50, 50, 12, 46};
    constexpr uint8_t kDefaultCp[Ws::kHops] = {14, 16, 84, 56, 10, 24, 15, 19};
    constexpr uint8_t kDefaultCpBf16[Ws::kHops] = {16, 10, 38, 56, 24, 26, 13, 23};
    constexpr uint8_t kDefaultSpread17Bf16[Ws::kHops] = {74, 40, 136, 64, 8, 0, 26, 68};
    constexpr uint8_t kDefaultCpProj[Ws::kHops] = {14, 16, 20, 58, 12, 24, 24, 16};
    constexpr uint8_t kDefaultCpProjBf16[Ws::kHops] = {10, 14, 18, 60, 24, 26, 24, 20};
    constexpr bool kProj = CP && CpProjIn<H, I>::value > 0;
    const uint32_t w0 = s_dl[0], w1 = s_dl[1];
#pragma unroll
    for (int h = 0; h < Ws::kHops; h++) {
      const uint32_t v = ((h < 4 ? w0 : w1) >> (8 * (h & 3))) & 0xffu;
      c.dl[h] = v ? (uint8_t)(v - 1)
                  : CP ? (kProj ? (WD == SK_WD_BF16 ? kDefaultCpProjBf16[h] : kDefaultCpProj[h])
                                : (WD == SK_WD_BF16 ? kDefaultCpBf16[h] : kDefaultCp[h]))
                       : (CfgW<H, I, W, V, CP, WD>::kSpread
                              ? (H == 1024 ? kDefaultSpread06[h]
                                           : (WD == SK_WD_BF16    ? kDefaultSpread17Bf16[h]
                                              : WD == SK_WD_I8G32 ? kDefaultSpread17G32[h]
                                                                  : kDefaultSpread[h]))
                              : kDefault[h]);
    }
  }
  c.trace = s_trace ? (uint64_t*)((char*)ws + Ws::kTrace) : nullptr;
  if constexpr (PAIRK) {
    if (wave == W) ctl_pair_pass<H, I, W, V, CP>(c, S, lane);
    else compute_pair<H, I, W, V, CP, WD, KEEP>(c, S, wave, tid, lane);
  } else {
    if (wave == W) run_control<H, I, W, V, CP, SMP, F16, CfgW<H, I, W, V, CP, WD>::kSingle>(c, S, lane);
    else run_compute<H, I, W, V, CP, SMP, WD, KEEP, F16>(c, S, wave, tid, lane);
  }
  // ---- end of launch: epoch base and launch count (workgroup 0; every workgroup finished its census) --------
  if (c.g == 0 && tid == 0) {
    st_u32_dev(ws, Ws::kTick, c.base + (uint32_t)(PAIRK ? 1 : n_frames) * c.tpf);
    st_u32_dev(ws, Ws::kLaunch, ld_u32_dev(ws, Ws::kLaunch) + 1u);
  }
}
// First launch of an instantiation on a device: raise its LDS limit and check that the 256 workgroups can all be
// resident at once, one per CU (every exchange waits for all of them; a device with fewer CUs, or one whose CUs
// cannot hold a workgroup, would only surface as poll timeouts). Done once per device and instantiation; a failure
// is reported every time and retried on the next call.
constexpr int kMaxDevices = 64;
template <int H, int I, int W, int V, bool CP, bool SMP, int WD, bool KEEP, bool PAIRK, bool F16>
int prepare_kernel(size_t lds) {
  static bool ready[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return sk_set_error(SK_EDEVICE, "sk_talker_frames: no current HIP device");
  if (ready[dev]) return SK_OK;
  const void* fn = (const void*)k_frames<H, I, W, V, CP, SMP, WD, KEEP, PAIRK, F16>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return sk_check_launch(e, "sk_talker_frames: raising the LDS limit");
  int cus = 0, per_cu = 0;
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return sk_check_launch(e, "sk_talker_frames: reading the CU count");
  if (cus != kWG) return sk_set_error(SK_EUNSUPPORTED, "sk_talker_frames: needs a 256-CU device (8 XCDs x 32)");
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, (W + 1) * 64, lds);
  if (e != hipSuccess) return sk_check_launch(e, "sk_talker_frames: occupancy query");
  if (per_cu < 1)
    return sk_set_error(SK_EUNSUPPORTED, "sk_talker_frames: a CU cannot hold one workgroup of the frame kernel, so the "
                                         "256 workgroups cannot be co-resident");
  ready[dev] = true;
  return SK_OK;
}
template <int H, int I, int W, int V, bool CP, bool SMP, int WD, bool KEEP, bool PAIRK = false, bool F16 = false>
int launch_kernel(const sk_talker_desc* d, const CpArgs& cp, int n_frames, hipStream_t st) {
  constexpr size_t need = SMP ? kPickShared<H, I, W, V, CP> + sizeof(PickShared)
                              : sizeof(Lds<H, I, W, V, CP>) + (PAIRK ? sizeof(LdsPair<H, I>) : 0);
  const size_t lds = need < 96 * 1024 ? 96 * 1024 : need;  // one workgroup per CU
  const int rc = prepare_kernel<H, I, W, V, CP, SMP, WD, KEEP, PAIRK, F16>(lds);
  if (rc != SK_OK) return rc;
  hipLaunchKernelGGL((k_frames<H, I, W, V, CP, SMP, WD, KEEP, PAIRK, F16>), dim3(kWG), dim3((W + 1) * 64), lds, st, *d, cp,
                     n_frames);
  return sk_check_launch(hipGetLastError(), "sk_talker_frames");
}
// KEEP: the layer weights are loaded through the caches instead of as non-temporal streams (the code predictor
// with keep_layers; the heads and every talker weight stream).
template <int H, int I, int W, int V, bool CP, int WD = SK_WD_I8ROW, bool KEEP = false>
int launch_frames(const sk_talker_desc* d, const CpArgs& cp, int n_frames, hipStream_t st) {
  if (d->max_len > Cfg<H, I, W, V, CP>::kMaxLen) return sk_set_error(SK_EUNSUPPORTED, "sk_talker_frames: max_len too long");
  if constexpr (CP && CpProjIn<H, I>::value == 0) {
    if (cp.pair) {  // the paired pass first (no head: greedy and sampled launches share it)
      const int rc = launch_kernel<H, I, W, V, CP, false, WD, KEEP, true>(d, cp, n_frames, st);
      if (rc != SK_OK) return rc;
    }
  } else if constexpr (CP) {
    if (cp.pair) return sk_set_error(SK_EUNSUPPORTED, "sk_cp_frame: a projected code predictor runs unpaired");
  }
  if constexpr (CP) {
    if (d->max_len <= 16)  // the code predictor's 16 positions: the whole-cache attention of F16
      return d->do_sample ? launch_kernel<H, I, W, V, CP, true, WD, KEEP, false, true>(d, cp, n_frames, st)
                          : launch_kernel<H, I, W, V, CP, false, WD, KEEP, false, true>(d, cp, n_frames, st);
  }
  return d->do_sample ? launch_kernel<H, I, W, V, CP, true, WD, KEEP>(d, cp, n_frames, st)
                      : launch_kernel<H, I, W, V, CP, false, WD, KEEP>(d, cp, n_frames, st);
}

}  // namespace
