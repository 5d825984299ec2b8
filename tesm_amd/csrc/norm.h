// Residual add + RMSNorm of the TESM block: arguments shared by the kernel and the C-ABI layer.
#pragma once

#include "tesm_hip_internal.h"

namespace tesm {

constexpr int64_t kNormMaxD = 16384;

struct NormArgs {
  int dt = 0;                   // module dtype: x, weight, y
  int64_t M = 0, D = 0;
  float eps = 1e-5f;
  const void* x = nullptr;      // (M, ld_x)
  int64_t ld_x = 0;
  const void* res = nullptr;    // optional (M, ld_res) residual in res_dt
  int res_dt = 0;
  int64_t ld_res = 0;
  void* res_out = nullptr;      // optional (M, ld_res_out) x + residual in res_out_dt (may alias res)
  int res_out_dt = 0;
  int64_t ld_res_out = 0;
  const void* weight = nullptr; // (D)
  void* y = nullptr;            // optional (M, ld_y) normalised rows
  int64_t ld_y = 0;
  int8_t* q = nullptr;          // optional (M, ldq) int8 codes of y, layout 1, zero padded to ldq
  int64_t ldq = 0;
  float* s_x = nullptr;         // (M) code scales
  int32_t* rowsum = nullptr;    // (M) code sums
  float bit_eps = 1e-5f;
};

int launch_add_rmsnorm(const NormArgs& a, hipStream_t st);

}  // namespace tesm
