// Internal launchers shared between the kernel sources and the C-ABI layer.
#pragma once

#include <algorithm>

#include "common.h"

namespace tesm {

typedef int v4i __attribute__((ext_vector_type(4)));

// zero_p / zero_n: an int range the kernel also clears (for a later kernel of the same stream).
int launch_quant_act(const void* x, int dt, int64_t M, int64_t K, int64_t ldx, float eps, int layout, int8_t* q,
                     int64_t ldq, float* s_x, int32_t* rowsum, hipStream_t st, int* zero_p = nullptr,
                     int64_t zero_n = 0);
// The codes of a second matrix of the same shape and row pitch in the same launch (layout 1), e.g.
// tanh(E) and C: one launch instead of two.
struct QuantSet {
  const void* x = nullptr;
  int8_t* q = nullptr;
  float* s = nullptr;
  int32_t* rs = nullptr;
};
int launch_quant_act2(const void* x0, const void* x1, int dt, int64_t M, int64_t K, int64_t ldx, float eps,
                      int8_t* q0, int8_t* q1, int64_t ldq, float* s0, float* s1, int32_t* rs0, int32_t* rs1,
                      hipStream_t st);
int launch_absmean(const void* w, int dt, int64_t n, float eps, double* ws, float* s_w, float* c_w, hipStream_t st);
int launch_pack(const void* w, int dt, int64_t N, int64_t K, int64_t ldw, const float* s_w, int per_row,
                uint8_t* packed, int64_t ldp, hipStream_t st);
int launch_stream_copy(void* dst, const void* src, int64_t bytes, hipStream_t st);
int launch_unpack(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* codes, int64_t ldc,
                  hipStream_t st);

// One INT2 x INT8 product  out = (A_codes . W_codes) / s_x * c_w (+ bias).
struct LinearOperand {
  const int8_t* q = nullptr;     // (M, ldq) activation codes, layout 1, zero padded to Kp
  int64_t ldq = 0;
  const float* s_x = nullptr;    // (M) activation scales
  const int32_t* rowsum = nullptr;  // (M) sum of activation codes
  const uint8_t* w = nullptr;    // (N, ldw) packed INT2 weights, padded with code 1 to Kp
  int64_t ldw = 0;
  const float* c_w = nullptr;    // dequantized +1 weight value: scalar, or (N) if c_w_per_row
  int c_w_per_row = 0;
};

// Epilogues of the GEMM/GEMV.
enum Epilogue : int {
  kEpiStore = 0,       // out = rnd(v (+ bias))
  kEpiOutputGate = 1,  // out = rnd(rnd(local + rnd(sigmoid(gate) * sp)) + ep), two products (sp, ep)
  kEpiSwiGLU = 2,      // out = rnd(rnd(silu(rnd(g))) * rnd(u)), two products (g, u) of one activation
  kEpiGates = 3,       // kEpiStore with the MIMO scan's gate activations on three column regions
};

// Epilogues that combine two products (op[0], op[1]) computed over the same output tile.
constexpr bool epi_dual(int epi) { return epi == kEpiOutputGate || epi == kEpiSwiGLU; }

struct LinearArgs {
  LinearOperand op[2];  // op[1] used only by the two-product epilogues
  int64_t M = 0, N = 0, Kp = 0;
  const void* bias = nullptr;  // (N) in out dtype, kEpiStore only
  void* out = nullptr;
  int64_t ldo = 0;
  int out_dt = 0;
  int epilogue = kEpiStore;
  const void* local = nullptr;  // kEpiOutputGate: (M, ld_local) and raw gate (M, ld_gate), out dtype
  int64_t ld_local = 0;
  const void* gate = nullptr;
  int64_t ld_gate = 0;
  int32_t* acc_dump = nullptr;  // optional (M, N) signed int32 accumulators of op[0]
  // kEpiGates (tesm_mimo.py:957-986, the gates of the MIMO state scan), on the rounded product p of
  // column n: [act_n0, act_n0 + act_w) -> rnd(tanh(p)) (the state value), the next act_w columns ->
  // rnd(sigmoid(rnd(p + act_bias[c]))) (the decay, c counted from that region's start), the next
  // act_w -> rnd(sigmoid(p)) (the write gate); other columns are stored as kEpiStore stores them.
  // act_n0 and act_w are multiples of 32, act_bias is (act_w) in the out dtype; M > 32, no bias.
  int64_t act_n0 = 0, act_w = 0;
  const void* act_bias = nullptr;
};

int launch_linear(const LinearArgs& a, hipStream_t st);

// Raw activations for a product that quantizes them itself (x: (M, ldx) in dt, K values per row).
struct FusedQuantIn {
  const void* x = nullptr;
  int64_t ldx = 0, K = 0;
  float eps = 0.0f;
  int dt = 0;
};
// Store-epilogue product with the per-token activation quantization fused in (one launch instead
// of quant_act + product); linear_fq_ok tells whether the sizes allow it.  Operand 0's q / s_x /
// rowsum are not read.
bool linear_fq_ok(const LinearArgs& a);
int launch_linear_fq(const LinearArgs& a, const FusedQuantIn& f, hipStream_t st);

// Per-token int8 codes of the output-gate result y (the out_proj input), written instead of y.
struct RowQuant {
  int8_t* q = nullptr;   // (M, ldq) layout-1 codes
  int64_t ldq = 0;
  float* s = nullptr;    // (M) scales
  int32_t* rs = nullptr; // (M) code sums
  float eps = 1e-5f;
  void* y = nullptr;     // optional (M, ldy) y itself, in the output dtype
  int64_t ldy = 0;
};

// Output gate (kEpiOutputGate operands) with the whole row per workgroup; N <= 1024.
int launch_gate_rowq(const LinearArgs& a, const RowQuant& o, hipStream_t st);

// Output gate and out_proj in one launch: each 32-row workgroup quantizes its y rows into LDS and runs
// out_proj (K = N = d_model) on them, writing out (M, ldout) in the output dtype.  o.q / o.s / o.rs are
// written only when o.q is set (decision taps).  Returns -1 (nothing launched) where the sizes do not
// allow it (bf16, per-tensor weight scales, d_model 768, the 32-row gate's other limits).
int launch_gate_out(const LinearArgs& a, const RowQuant& o, const LinearOperand& out_proj, void* out, int64_t ldout,
                    hipStream_t st);

}  // namespace tesm
