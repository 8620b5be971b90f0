// Host-side helpers shared by the C-ABI entry points (not exported beyond the library).
#pragma once
#include <hip/hip_runtime.h>
#include "sokutou_amd.h"

// Records `msg` as the thread's last error and returns `rc` (so callers can `return sk_set_error(...)`).
int sk_set_error(int rc, const char* msg);
// Maps a launch status to SK_OK / SK_ELAUNCH, recording the HIP error string.
int sk_check_launch(hipError_t e, const char* where);
// Launches the frame kernel of the 1.7B talker shape (hidden 2048, intermediate 6144, 4 compute waves; i8row or
// i8g32 weights) on a validated descriptor; a translation unit of its own (frame17.hip), called by sk_talker_frames.
int sk_talker_frames_2048(const sk_talker_desc* d, int n_frames, hipStream_t st);
// Launches the frame kernel of the 0.6B talker shape with i8g32 weights (frame_g32.hip) on a validated descriptor.
int sk_talker_frames_g32(const sk_talker_desc* d, int n_frames, hipStream_t st);
// The 1.7B shape's i8g32 kernel (frame17_g32.hip), called by sk_talker_frames_2048.
int sk_talker_frames_2048_g32(const sk_talker_desc* d, int n_frames, hipStream_t st);
// The 1.7B shape's bf16 kernel (frame17_bf16.hip), called by sk_talker_frames_2048.
int sk_talker_frames_2048_bf16(const sk_talker_desc* d, int n_frames, hipStream_t st);
// The 0.6B talker shape with bf16 weights (frame_bf16.hip), called by sk_talker_frames.
int sk_talker_frames_bf16(const sk_talker_desc* d, int n_frames, hipStream_t st);
// sk_cp_frame with i8g32 or bf16 weights (frame_cp_g32.hip, frame_cp_bf16.hip; the arguments already checked by
// sk_cp_frame).
int sk_cp_frame_g32(const sk_cp_desc* d, hipStream_t st);
int sk_cp_frame_bf16(const sk_cp_desc* d, hipStream_t st);
// sk_cp_frame of a projected code predictor (proj_in 2048; frame_cp_proj.hip), any of the three weight formats.
int sk_cp_frame_proj(const sk_cp_desc* d, hipStream_t st);

#define SK_ALIGNED16(p) ((((uintptr_t)(p)) & 15u) == 0)
