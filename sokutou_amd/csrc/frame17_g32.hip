// The persistent frame kernel for the 1.7B talker (hidden 2048, intermediate 6144, 4 compute waves) with i8g32
// weights, the reference's int8 format (one fp16 scale per 32 weights of a row, qwen3/kernels.py:425-447; applied
// per 16-weight chunk inside the dots). The shape's traits as in frame17.hip (weights one exchange before their
// use, shared lane offsets: the group scales load through the same shared offset as their weights). A translation
// unit of its own, so the i8row kernels' module keeps its generated code.
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

int sk_talker_frames_2048_g32(const sk_talker_desc* d, int n_frames, hipStream_t st) {
  const CpArgs none{};
  return launch_frames<kH, kI, 4, kTalkerV, false, SK_WD_I8G32>(d, none, n_frames, st);
}
