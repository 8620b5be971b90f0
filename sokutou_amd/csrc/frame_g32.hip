// The persistent frame kernel for the 0.6B talker (hidden 1024, intermediate 3072) with i8g32 weights, the
// reference's int8 format (one fp16 scale per 32 weights of a row, qwen3/kernels.py:425-447). A translation unit of
// its own, so the i8row kernels' module (frame.hip) keeps the code it was tuned with; the kernel is frame_impl.h's
// with the group scales applied per 16-weight chunk inside the dots.
#include "frame_impl.h"

int sk_talker_frames_g32(const sk_talker_desc* d, int n_frames, hipStream_t st) {
  const CpArgs none{};
  return launch_frames<1024, 3072, 4, kTalkerV, false, SK_WD_I8G32>(d, none, n_frames, st);
}
