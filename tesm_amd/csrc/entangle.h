// Local-window ternary entanglement arguments shared by the kernels and the layer drivers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace tesm {

// One RoPE'd pair (x[i], x[i + R/2]) rotated by (c, s), rounded like the reference (tesm.py:789-793).
template <int DT>
__device__ __forceinline__ void rope_pair(float xa, float xb, float2 cs, float& o1, float& o2) {
  o1 = rnd<DT>(rnd<DT>(xa * cs.x) - rnd<DT>(xb * cs.y));
  o2 = rnd<DT>(rnd<DT>(xa * cs.y) + rnd<DT>(xb * cs.x));
}

// RoPE table: tab[(t * (R/2) + i)] = (cos, sin) of (pos_offset + t) * inv_freq[i], rounded to dt.
int launch_rope_table(float2* tab, int64_t L, int64_t R, int64_t pos_offset, double base, int dt, hipStream_t st);

struct EntArgs {
  int dt = 0;         // dtype of q, k, states and outputs
  int mimo = 0;       // 0: SISO window (tesm.py:921-952); 1: MIMO window (tesm_mimo.py:525-588)
  int64_t B = 0, L = 0, H = 1, R = 0, D = 0;
  int64_t W = 0;      // configured window (entanglement_window)
  // element (b, t, h, r) of q/k at ptr[(b*L + t)*ld + h*R + r]; raw (pre-RoPE) values
  const void* q = nullptr;
  int64_t ld_q = 0;
  const void* k = nullptr;
  int64_t ld_k = 0;
  const float2* rope = nullptr;  // (L, R/2) table; positions 0..L-1
  const void* q_add = nullptr;   // optional (b, t, h, r) added to RoPE(q), ld_qadd
  int64_t ld_qadd = 0;
  const float* bias = nullptr;   // (H, W) window bias as floats holding dt values
  float thr = 0.0f;              // threshold already rounded to dt
  float ent_scale = 0.0f;        // entanglement_scale
  // element (b, t, h, d) of states at S[(b*L + t)*ld_s + h*D + d]
  const void* S = nullptr;
  int64_t ld_s = 0;
  // outputs, element (b, t, h, d) at ptr[(b*L + t)*ld_out + h*D + d]; each may be null
  void* avg = nullptr;     // window average (tesm.py:952 `out`)
  void* e_tanh = nullptr;  // tanh(S + scale*(avg - S))
  void* c_out = nullptr;   // (S + scale*(avg - S)) - S
  void* e_out = nullptr;   // S + scale*(avg - S)
  int64_t ld_out = 0;
  int8_t* tern = nullptr;  // optional ternary map (b, t, h, w) over the effective window
  float* wts = nullptr;    // workspace (B, L, H, W_eff) floats: normalised window weights
  // fused per-token int8 quantization of tanh(E) and C (the state_proj / ent_proj inputs);
  // codes in layout 1, rows of ldq = kpad(H*D) bytes.  Used when q_te != nullptr.
  int8_t* q_te = nullptr;
  float* s_te = nullptr;
  int32_t* rs_te = nullptr;
  int8_t* q_c = nullptr;
  float* s_c = nullptr;
  int32_t* rs_c = nullptr;
  int64_t ldq = 0;
  float eps = 1e-5f;
};

// True when launch_local_ent can produce the quantized outputs in one fused kernel.
bool ent_fused_ok(const EntArgs& a);

int64_t ent_ws_bytes(int64_t B, int64_t L, int64_t H, int64_t W);
int launch_local_ent(const EntArgs& a, hipStream_t st);

}  // namespace tesm
