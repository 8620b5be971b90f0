// The persistent frame kernel for the 1.7B talker (hidden 2048, intermediate 6144, 4 compute waves) with bf16
// weights, the reference's Qwen3Kernels default (qwen3/kernels.py:487; no scales). The shape's traits as in
// frame17.hip: every stage's weights are loaded one exchange before their use and gate/up is split over two
// exchanges. At twice the bytes of int8 a stage's rows take twice the registers (the gate/up half of a wave: 6 rows
// of 2048 bf16 weights, 96 registers); the kernel spills 44 registers (47 sampled), against 2 for i8row. A
// translation unit of its own, so the int8 kernels' modules keep their generated code.
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

}  // namespace

int sk_talker_frames_2048_bf16(const sk_talker_desc* d, int n_frames, hipStream_t st) {
  const CpArgs none{};
  return launch_frames<kH, kI, 4, kTalkerV, false, SK_WD_BF16>(d, none, n_frames, st);
}
