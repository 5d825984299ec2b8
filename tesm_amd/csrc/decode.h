// TESM_SISO / TESMMIMO_Optimized decode step and prefill cache fill: arguments shared by the kernels and
// the drivers.
#pragma once

#include "entangle.h"

namespace tesm {

// One decode step of the entanglement block for B rows (one token each) and H heads (SISO: H = 1).
// Per-head data: state / new state / cross query rows b*H + h; proj slices at o_* + h*D (h*R for q, k);
// decay bias (H, D); window bias (H, W); rings (B, W, H, R) and (B, W, H, D).
struct DecodeArgs {
  int dt = 0;                  // layer dtype
  int cdt = 0;                 // ring buffer dtype
  int64_t B = 0, R = 0, D = 0, W = 0;
  int64_t H = 1;
  int64_t chunk = 0;           // channels per workgroup (set by launch_decode_ent)
  int vec4 = 0;                // ring states may be read four at a time (set by launch_decode_ent)
  int64_t pos = 0;             // RoPE position of this token (seq_pos before the step)
  int64_t slot = 0;            // ring slot written by this step (cache_idx)
  int64_t valid = 0;           // min(seq_pos + 1, W)
  int full = 0;                // valid >= W
  // in_proj output (B, ld_proj) in dt; column offsets of the sv, decay, write, q and k slices
  const void* proj = nullptr;
  int64_t ld_proj = 0, o_sv = 0, o_decay = 0, o_write = 0, o_q = 0, o_k = 0;
  const float2* rope = nullptr;     // table whose row `pos` holds this token's (cos, sin)
  const void* decay_bias = nullptr; // (D) dt
  const float* bias = nullptr;      // (W) window bias, dt values as floats
  const void* q_add = nullptr;      // optional (B*H, ld_qadd) cross-layer query in dt
  int64_t ld_qadd = 0;
  float thr = 0.0f, ent_scale = 0.0f, eps = 1e-5f;
  const double* state = nullptr;    // (B, H, D) float64 before the step
  double* state_out = nullptr;      // (B, H, D) float64 after the step (may equal state)
  void* k_cache = nullptr;          // (B, W, H, R) cdt
  void* v_cache = nullptr;          // (B, W, H, D) cdt
  void* new_state = nullptr;        // optional (B, H, D) dt: the step's state (next layer's cross state)
  // H > 1: tanh(E) and C in dt, element (b, h, d) at te_out[b*ld_out + h*D + d]
  void* te_out = nullptr;
  void* c_out = nullptr;
  int64_t ld_out = 0;
  // H == 1: int8 codes (layout 1), scales and row sums of tanh(E) and C = E - S
  int8_t* q_te = nullptr;
  float* s_te = nullptr;
  int32_t* rs_te = nullptr;
  int8_t* q_c = nullptr;
  float* s_c = nullptr;
  int32_t* rs_c = nullptr;
  int64_t ldq = 0;
  // optional (B, H, W) int8 ternary decisions at the padded window positions (reference read order)
  int8_t* tern = nullptr;
  // optional device {seq_pos, cache_idx}: read at run time instead of pos / slot / valid / full (RoPE
  // rows clamped to rope_rows - 1); launch_decode_advance moves it to the next step
  const int64_t* step_pos = nullptr;
  int64_t rope_rows = 0;
};

int64_t decode_lds_bytes(int64_t R, int64_t CW);
int launch_decode_ent(const DecodeArgs& a, hipStream_t st);
// step_pos = {seq_pos + 1, (cache_idx + 1) % W}: the device-side position of a graph-replayed step
int launch_decode_advance(int64_t* step_pos, int64_t W, hipStream_t st);

// Ring buffers after a prefill of L tokens: the last min(L, W) RoPE'd keys and states.
struct CacheFillArgs {
  int dt = 0, cdt = 0;
  int sdt = -1;                     // states dtype (-1: dt)
  int64_t B = 0, L = 0, H = 1, R = 0, D = 0, W = 0;
  const void* k = nullptr;          // raw (pre-RoPE) keys, element (b, t, h, r) at k[(b*L + t)*ld_k + h*R + r]
  int64_t ld_k = 0;
  const float2* rope = nullptr;     // (L, R/2) table, positions 0..L-1
  const void* states = nullptr;     // (b, t, h, d) at states[(b*L + t)*ld_states + h*D + d]
  int64_t ld_states = 0;
  const float* vscale = nullptr;    // optional per-channel factor (H*D) applied to the states
  void* k_cache = nullptr;          // (B, W, H, R) cdt
  void* v_cache = nullptr;          // (B, W, H, D) cdt
};

int launch_cache_fill(const CacheFillArgs& a, hipStream_t st);

}  // namespace tesm
