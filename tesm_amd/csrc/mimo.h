// TESMMIMO_Optimized pieces around the shared scan / window-score kernels.
#pragma once

#include "entangle.h"

namespace tesm {

// c[h, d] = sum_r mimo_x[h,r,d]^2 * mimo_o[h,r,d] and x0sq[h, d] = mimo_x[h,0,d]^2 in float32.
int launch_mimo_coef(const void* mimo_x, const void* mimo_o, int dt, int64_t H, int64_t Rm, int64_t D, float* coef,
                     float* x0sq, hipStream_t st);

// Window mix of the rank-free states S (float32, (B, L, H*D)) with the window weights of
// ent_scores_kernel (MIMO form, (B, L, H, W)), entangled state E = S + scale (A - S) and
// C = E - S in float32, then tanh(E * c) and C * c rounded to dt, (B*L, H*D) each.
struct MimoMixArgs {
  int dt = 0;
  int64_t B = 0, L = 0, H = 0, D = 0, W = 0;
  const float* S = nullptr;
  const float* wts = nullptr;
  const float* coef = nullptr;
  float ent_scale = 0.0f;
  void* te = nullptr;
  void* cc = nullptr;
};
int launch_mimo_mix(const MimoMixArgs& a, hipStream_t st);

// Entanglement statistics of tesm_mimo.py:458-523 (window > 0 branch), taken on the RoPE'd q and k
// of the first S = min(L, 64) positions: for every complete window v in [0, S - W + 1), head h and
// slot w, score = fl(fl(sum_r fl(q[W-1+v, h, r] * k[v+w, h, r])) / sqrt(R)) (no local bias) and its hard
// ternary against +-thr, written in dt as (B, V, H, W); counts[b] = (#positive, #negative, #zero).
struct MimoStatsArgs {
  int dt = 0;
  int global = 0;                // 1: global branch (:469-482): S = min(L, 32) positions, all pairs,
                                 //    one score per pair summed over heads, output (B, S, S)
  int64_t B = 0, L = 0, H = 0, R = 0;
  int64_t W = 0;                 // window actually used: min(entanglement_window, L)
  int64_t S = 0;                 // sampled positions: min(L, 64); V = S - W + 1 >= 1
  const void* q = nullptr;       // (b, t, h, r) at q[(b*L + t)*ld_q + h*R + r], raw (pre-RoPE)
  int64_t ld_q = 0;
  const void* k = nullptr;
  int64_t ld_k = 0;
  const float2* rope = nullptr;  // (L, R/2) cos/sin rounded to dt
  float sqrt_r = 0.0f;           // float(sqrt(R)), the divisor
  float thr = 0.0f;              // threshold rounded to dt
  void* ternary = nullptr;       // (B, V, H, W) in dt
  int32_t* counts = nullptr;     // (B, 3)
};
int launch_mimo_stats(const MimoStatsArgs& a, hipStream_t st);

// Rank-0 final state h[b, c] = float64(S[b, L-1, c] * x0sq[c]) and, optionally, its float32 copy.
int launch_mimo_final(const float* S, const float* x0sq, int64_t B, int64_t L, int64_t C, double* h_final,
                      float* last, hipStream_t st);

}  // namespace tesm
