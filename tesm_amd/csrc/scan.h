// State-scan arguments shared by the scan kernels and the fused layer drivers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tesm {

struct ScanArgs {
  // 0: decay/update given; 1: gates from raw projection slices; 2: gates already applied by the
  // producer (decay = sigmoid(x + bias), write = sigmoid, sv = tanh, each rounded to dt), so the scan
  // forms only update = write * sv
  int mode = 0;
  int dt = 0;          // input dtype (0 f32, 1 bf16)
  int out_dt = 0;      // states dtype
  int clamp = 1;       // 1: SISO closed-form clamp semantics (1e-12); 0: plain recurrence (MIMO)
  int round_update = 1;  // modes 1, 2: round write*tanh(sv) to dt (SISO) or keep fp32 (MIMO); in
                         // these modes clamp and round_update must agree (the SISO and MIMO semantics)
  int64_t B = 0, L = 0, C = 0;
  int64_t cs = 16;     // reference chunk size (state_scan_chunk_size)
  // token-major inputs: element (b, t, c) at ptr[(b*L + t)*ld + c]
  const void* decay = nullptr;   // mode 0: decay; mode 1: raw decay slice; mode 2: decay gate
  int64_t ld_decay = 0;
  const void* update = nullptr;  // mode 0: update; mode 1: raw write slice; mode 2: write gate
  int64_t ld_update = 0;
  const void* sv = nullptr;      // mode 1: raw state_value slice; mode 2: tanh(state_value)
  int64_t ld_sv = 0;
  const void* decay_bias = nullptr;  // mode 1: (C) in dt
  const double* h0 = nullptr;    // (B, C) initial state or null
  void* states = nullptr;        // (b, t, c) at states[(b*L + t)*ld_states + c], out_dt
  int64_t ld_states = 0;
  double* h_final = nullptr;     // (B, C) final state or null
  // 1: the single-pass scan's flags and span counters in the workspace are already zero (the caller
  // cleared the range scan_lb_clear_range names, in an earlier kernel of the same stream)
  int flags_clear = 0;
};

int64_t scan_chunk_len(int64_t L, int64_t cs);
int64_t scan_ws_bytes(int64_t B, int64_t L, int64_t C, int64_t cs);
int launch_scan(const ScanArgs& a, void* ws, int64_t ws_bytes, hipStream_t st);
// The int range of the workspace the single-pass scan needs zero at its start (*n = 0 when that
// pass will not run for these sizes and this workspace).
// Status word of the look-back scan on the current device (bit 0: a poll gave up); synchronous.
int scan_status(unsigned* out, int clear);
// Poll limit of later look-back launches (< 0: give up at once; a test of the failure report).
void scan_set_spin_limit(int limit);
void scan_lb_clear_range(int64_t B, int64_t L, int64_t C, int64_t cs, void* ws, int** p, int64_t* n);

}  // namespace tesm
