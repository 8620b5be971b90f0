// The 1.7B talker's instantiations of the persistent kernel (hidden 2048, intermediate 6144) with 4 compute waves.
//
// Four compute waves leave the control wave 256 registers, enough to poll every exchange straight into registers
// (the 0.6B kernels' polls); a full layer of 1.7B weights does not fit in the compute waves' registers beside the
// rest, so each stage's weights are loaded one exchange before their use (SpreadLate; issuing o and gate/up
// together after the attention measured 28.4 us per layer), except the first half of the gate/up rows, which goes
// out with o (SplitGateUp: 25 MB of gate/up weights per layer take longer than one exchange to stream; 24.2
// against 25.2 us per layer). Every cell, weight-row and cache access of this shape
// keeps its lane part in one shared vector offset and its uniform part in the scalar offset (LaneOffsetPolls):
// with a vector address per access the waves spilled ~140 addresses and reloaded them from scratch on every
// exchange; with the shared offsets nothing spills. Measured on the 64-frame 1.7B workload: 25.3 us per layer,
// against 38.8 us for 8 compute waves with polls staged through LDS (the 168-register budget of 9 waves) and 69 us
// for 8 compute waves with register polls (instantiations since deleted).
#include "frame_impl.h"

namespace {

constexpr int kH = 2048, kI = 6144;
template <>
struct SpreadLate<kH, kI> {
  static constexpr bool value = true;
};
template <>
struct LaneOffsetPolls<kH> {
  static constexpr bool value = true;
};
template <>
struct SplitGateUp<kH, kI> {
  static constexpr bool value = true;
};
static_assert(Cfg<kH, kI, 4, kTalkerV, false>::kMaxLen >= 2048, "1.7B caches up to 2048 positions");

}  // namespace

int sk_talker_frames_2048(const sk_talker_desc* d, int n_frames, hipStream_t st) {
  const CpArgs none{};
  if (d->wd == SK_WD_I8G32) return sk_talker_frames_2048_g32(d, n_frames, st);
  if (d->wd == SK_WD_BF16) return sk_talker_frames_2048_bf16(d, n_frames, st);
  return launch_frames<kH, kI, 4, kTalkerV, false>(d, none, n_frames, st);
}
