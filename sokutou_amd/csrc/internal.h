// Host-side helpers shared by the C-ABI entry points (not exported beyond the library).
#pragma once
#include <hip/hip_runtime.h>
#include "sokutou_amd.h"

// Records `msg` as the thread's last error and returns `rc` (so callers can `return sk_set_error(...)`).
int sk_set_error(int rc, const char* msg);
// Maps a launch status to SK_OK / SK_ELAUNCH, recording the HIP error string.
int sk_check_launch(hipError_t e, const char* where);

#define SK_ALIGNED16(p) ((((uintptr_t)(p)) & 15u) == 0)
