// zm_host.hpp -- host helpers shared by the translation units of
// libzeromoe_hip.so: the thread-local error text behind zm_last_error(), the
// per-device IQ2_XXS grid and the MUL_MAT_ID hook launch counter.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zm {

// record the reason of a rejected call; returns -1
int fail(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
// the current device's IQ2_XXS grid (256 x u64, device memory), set up on first use
int device_grid(const uint64_t **grid);
// the current device's lookup table of a weight type: the IQ4_XS value table
// (16 x i8) for T_IQ4_XS, the IQ2_XXS grid otherwise
int device_table(int type, const uint64_t **table);
// one more executed MUL_MAT_ID hook launch (zm_mul_mat_id_launches)
void count_mmid_launch();

}  // namespace zm

#define HIP_OK(call)                                                                  \
  do {                                                                                \
    hipError_t e_ = (call);                                                           \
    if (e_ != hipSuccess) return zm::fail("%s: %s", #call, hipGetErrorString(e_));    \
  } while (0)
