// Global (causal, full-history) ternary entanglement: TESM_SISO with entanglement_window = 0
// (tesm_ssm/modules/tesm.py:963-1063, torch branch 1040-1052) and TESMMIMO_Optimized's global branch
// (tesm_mimo.py:590-687, torch branch 655-687).
#pragma once

#include "entangle.h"

namespace tesm {

// Relative-position bias (tesm.py:970-982).  Positions are arange(L) in the layer dtype and the bias
// of a (query, key) pair is a function of rel = dt(pos_q - pos_k) alone, an integer-valued number in
// [0, 2L) for causal pairs; table[r] = that function at rel = r, a float holding a dt value:
//   ang_p = dt(r * freq_p), freq_p = dt(dt(p * pi) / 1000), p = 1 .. P
//   b = dt(dt(sum_p dt(dt(sin ang_p) * e_p)) + dt(sum_p dt(dt(cos ang_p) * e_p)))
//   table[r] = dt(dt(b * scale) + bias)
// embed (P), scale and bias are float32 arrays holding the parameters rounded to dt.
int launch_global_bias_table(int dt, int64_t n, const float* embed, int64_t P, const float* scale, const float* bias,
                             float* table, hipStream_t st);

struct GlobalArgs {
  int dt = 0;
  int mimo = 0;                  // 0: SISO (E = S + scale (A - S)); 1: MIMO (E = A, outputs scaled by coef)
  int64_t B = 0, L = 0, H = 1, R = 0, D = 0;  // q / k: H heads of R (RoPE per head); states: H*D channels
  const void* q = nullptr;       // (b, t, h, r) raw at q[(b*L + t)*ld_q + h*R + r]
  int64_t ld_q = 0;
  const void* k = nullptr;
  int64_t ld_k = 0;
  const float2* rope = nullptr;  // (L, R/2), positions 0..L-1
  const void* q_add = nullptr;   // optional SISO cross-layer query bias, added after RoPE
  int64_t ld_qadd = 0;
  const float* table = nullptr;  // bias table over rel in [0, 2L)
  float thr = 0.0f;              // rounded to dt
  float sqrt_div = 1.0f;         // float(sqrt(H*R))
  float ent_scale = 0.0f;
  const void* S = nullptr;       // states (b, t, c) at S[(b*L + t)*ld_s + c], c < H*D; dt (SISO) or f32 (MIMO)
  int64_t ld_s = 0;
  const float* coef = nullptr;   // MIMO: (H*D) rank merge factors
  void* e_tanh = nullptr;        // (b, t, c) at [(b*L + t)*ld_out + c], dt: tanh(E) (MIMO: tanh(E * coef))
  void* c_out = nullptr;         // E - S (MIMO: (E - S) * coef)
  int64_t ld_out = 0;
  int8_t* tern = nullptr;        // workspace (B, L, ldt) ternary decisions, ldt = round_up(L, 64); a row's
                                 // columns past its 64-key diagonal tile are left unwritten
  int32_t* count = nullptr;      // workspace (B, L) nonzero decisions per query
  uint16_t* states_t = nullptr;  // workspace (B, H*D, ldt) bf16 states transposed (bf16 SISO layers only)
  float* qr = nullptr;           // workspace (B, L, H*R) RoPE'd queries (+ cross-layer bias)
  float* kr = nullptr;           // workspace (B, L, H*R) RoPE'd keys
};

int64_t global_tern_pitch(int64_t L);
// bytes of the transposed-states workspace (zero where the states are float32)
int64_t global_states_t_bytes(int dt, int mimo, int64_t B, int64_t L, int64_t C);
int launch_global_ent(const GlobalArgs& a, hipStream_t st);

}  // namespace tesm
