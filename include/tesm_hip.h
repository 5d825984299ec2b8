/*
 * tesm_hip.h -- C-ABI of libtesm_hip.so, the gfx950 (MI355X) kernels behind kernel_backend='hip'.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers unless noted; every output and workspace is allocated by the
 *     caller.  No entry point allocates device memory or synchronises with the host.
 *   - `stream` is a hipStream_t (NULL = the null stream); work is queued asynchronously on it.
 *   - Element types: 0 = float32, 1 = bfloat16 (TESM_DT_*).  Sizes and leading dimensions are in
 *     elements unless named *_bytes.
 *   - Return 0 on success or a TESM_ERR_* code; tesm_hip_last_error() then describes the failure
 *     (thread-local, valid until the next call on the same thread).
 *   - Activation-code buffers are int8 (rows, ldq) with ldq a multiple of 16 and >= kpad(K); packed
 *     weights are uint8 (N, ldw) with ldw a multiple of 16 and >= kpad(K)/4 for the products.
 *     kpad(K) = tesm_hip_kpad(K) rounds K up to the 128-code GEMM tile; pad codes are 0 in
 *     activations and code 1 (value 0) in weights.
 *
 * Reference = WANGLILIN360/tesm.  Each declaration names the reference interface it replaces.
 */
#ifndef TESM_HIP_H_
#define TESM_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TESM_HIP_ABI_VERSION 9

#define TESM_DT_F32 0
#define TESM_DT_BF16 1

#define TESM_OK 0
#define TESM_ERR_INVALID_ARG 1
#define TESM_ERR_ALIGNMENT 2
#define TESM_ERR_UNSUPPORTED 3
#define TESM_ERR_LAUNCH 4
#define TESM_ERR_WORKSPACE 5

/* Library identity.  No reference counterpart (the reference loads a pybind11 module,
 * tesm_ssm/ops/cuda/__init__.py:19-48). */
int tesm_hip_abi_version(void);
const char* tesm_hip_last_error(void);
int64_t tesm_hip_kpad(int64_t K);

/* Launch log, a test and profiling aid with no reference counterpart: it names the kernel
 * instantiations a call selects.  tesm_hip_launch_log(1) clears the log and starts recording
 * "name<template args>\n" for every kernel launch of the process; (0) clears it and stops.
 * tesm_hip_launch_log_read copies the log into buf (NUL-terminated, cut to cap - 1 bytes), returns
 * its full length in bytes, and empties it when clear != 0.  Host-side only; thread-safe. */
int tesm_hip_launch_log(int enable);
int64_t tesm_hip_launch_log_read(char* buf, int64_t cap, int clear);

/* Streaming device copy of `bytes` bytes (16-byte vector loads and stores when both pointers are
 * 16-byte aligned), a measurement aid with no reference counterpart: the HBM bandwidth ceiling that
 * the bandwidth-bound kernels are compared with, and a known-size reference for byte counters. */
int tesm_hip_stream_copy(void* dst, const void* src, int64_t bytes, void* stream);

/* Device status word of the library's bounded waits on the current device, no reference
 * counterpart (the reference's kernels never wait on one another).  Bit 0 (TESM_STATUS_SCAN_GAVE_UP):
 * a single-pass scan's look-back poll gave up; the states of that span are NaN.  The kernels still
 * return, so a caller that wants certainty checks this word after its work.  Synchronises with the
 * device (a diagnostic, not for the hot path); clear != 0 zeroes the word after reading it.
 * tesm_hip_debug_scan_spin_limit sets the poll limit of later scans (default 1 << 20 rounds; a
 * negative limit gives up at once, which tests use to exercise the report). */
#define TESM_STATUS_SCAN_GAVE_UP 1u
int tesm_hip_device_status(uint32_t* status, int clear);
int tesm_hip_debug_scan_spin_limit(int limit);

/* Decision taps, a parity-test aid.  The reference's eval forward keeps its ternary decisions
 * (last_entanglement_map, tesm.py:716-744); its int8 codes are internal to BitLinear
 * (tesm.py:206-209).  While taps are set, each later call of tesm_hip_siso_prefill,
 * tesm_hip_siso_decode, tesm_hip_mimo_prefill and tesm_hip_mimo_decode also copies its discrete
 * decisions to these device buffers (any may be NULL):
 *   q_u/s_u, q_cs/s_cs, q_te/s_te, q_c/s_c, q_y/s_y: layout-1 int8 codes (M, kpad(K)) and scales (M)
 *     of the inputs of in_proj (u), cross_layer_q_proj (the cross-layer state; MIMO decode: B*n_heads
 *     rows), state_proj (tanh E), ent_proj (C) and out_proj (y); M = B*L (prefill) or B (decode),
 *     K = d_model for u and y, d_state for cs, d_state (SISO) or n_heads*d_state (MIMO) for te/c;
 *     tesm_hip_ffn_forward: q_u/s_u the codes of x (gate_proj / up_proj), q_h/s_h those of h
 *     (down_proj);
 *   tern: prefill with window > 0: SISO (B, L, min(window, L)), MIMO (B, L, n_heads, window), entry w
 *     deciding key t - W + 1 + w (W the window used); prefill with window == 0 (global): (B, L, P),
 *     P = L rounded up to 64, entry [b, i, j] deciding key j for query i (valid for j <= i);
 *     decode: (B, n_heads, window) at the reference's padded window positions, in its ring read
 *     order (SISO: n_heads = 1);
 *   wts: MIMO prefill with window > 0: float32 window weights tern / norm, (B*L, n_heads, window);
 *   S: MIMO prefill: the float32 rank-free states (B*L, n_heads*d_state) (rank r's are S * mimo_x[r]^2);
 *   te, c: the layer-dtype values of tanh(E) and C = E - S that state_proj / ent_proj quantize
 *     (MIMO: merged over the ranks), (M, K_te) row-major; set both or neither;
 *   yv: the layer-dtype output-gate values y that out_proj quantizes, (M, d_model).
 * Copies are queued on the call's stream.  With taps set, u and y are quantized by their own
 * kernels (the same codes as the products that quantize them inline).  Process-wide;
 * tesm_hip_debug_taps(NULL) stops. */
typedef struct tesm_hip_taps {
  int8_t* q_u;
  float* s_u;
  int8_t* q_cs;
  float* s_cs;
  int8_t* q_te;
  float* s_te;
  int8_t* q_c;
  float* s_c;
  int8_t* q_y;
  float* s_y;
  int8_t* q_h;
  float* s_h;
  int8_t* tern;
  float* wts;
  float* S;
  void* te;
  void* c;
  void* yv;
} tesm_hip_taps;

int tesm_hip_debug_taps(const tesm_hip_taps* taps);

/* Per-token int8 activation codes.  Replaces BitLinear.quantized_input
 * (tesm_ssm/modules/tesm.py:206-209): s_x[m] = 127 / max(amax_k |x[m,k]|, eps) evaluated as
 * reciprocal()*127 with the module dtype's rounding, q = clamp(rne(x * s_x), -128, 127).
 * layout 0 writes codes row-major; layout 1 writes them in the order the INT2 products read
 * (within each group of 16 codes, byte 4s+j holds code 4j+s).  rowsum[m] = sum_k q[m,k] (nullable). */
int tesm_hip_quant_act_i8(const void* x, int dt, int64_t M, int64_t K, int64_t ldx, float eps, int layout,
                          int8_t* q, int64_t ldq, float* s_x, int32_t* rowsum, void* stream);

/* Per-tensor absmean ternary scale.  Replaces the scale of BitLinear.quantized_weight
 * (tesm.py:212): s_w = 1 / max(mean|w|, eps) in the weight dtype; c_w = 1 / s_w (the dequantised
 * value of a +1 code, tesm.py:215).  ws: tesm_hip_absmean_ws_bytes() bytes of device scratch. */
int64_t tesm_hip_absmean_ws_bytes(void);
int tesm_hip_absmean_scale(const void* w, int dt, int64_t n, float eps, void* ws, float* s_w, float* c_w,
                           void* stream);

/* Ternary codes clamp(rne(w * s_w), -1, 1) packed four per byte (code+1 in bits 2i..2i+1 of byte
 * k/4, i = k%4).  Replaces pack_ternary_to_int2 (tesm_ssm/utils/int2_quantization.py:21-58) fed by
 * BitLinear.quantized_weight's codes (tesm.py:213-214).  s_w is a device scalar, or (N) if
 * per_row.  Bytes past ceil(K/4) up to ldp hold code 1. */
int tesm_hip_pack_w_i2(const void* w, int dt, int64_t N, int64_t K, int64_t ldw, const float* s_w, int per_row,
                       uint8_t* packed, int64_t ldp, void* stream);

/* Inverse of the packing.  Replaces unpack_int2_to_ternary (int2_quantization.py:68-93). */
int tesm_hip_unpack_w_i2(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* codes, int64_t ldc,
                         void* stream);

/* INT2 x INT8 BitLinear product out[m,n] = (sum_k q[m,k] * code[n,k]) / s_x[m] * c_w (+ bias[n]).
 * Replaces BitLinear._project_quantized / F.linear on the dequantised operands
 * (tesm.py:238-290) and the cuda_quantized_linear op (tesm_ssm/ops/cuda/__init__.py:128-139).
 * q: layout-1 codes (M, ldq), kpad(K) wide; packed: (N, ldw).  c_w: device scalar or (N) if
 * c_w_per_row.  bias: (N) in out_dt or NULL.  acc_dump: optional (M, N) exact int32 accumulators.
 * M <= 4 runs the bandwidth-bound GEMV; larger M the int8-MFMA GEMM. */
int tesm_hip_bitlinear_i2(const int8_t* q, int64_t ldq, const float* s_x, const int32_t* rowsum,
                          const uint8_t* packed, int64_t ldw, const float* c_w, int c_w_per_row, const void* bias,
                          int64_t M, int64_t N, int64_t K, void* out, int out_dt, int64_t ldo, int32_t* acc_dump,
                          void* stream);

/* BitLinear forward from raw activations: the per-token int8 codes of x (tesm_hip_quant_act_i8)
 * and the INT2 product (tesm_hip_bitlinear_i2) in one call.  Replaces BitLinear.forward
 * (tesm.py:287-290) for a packed weight.  x: (M, ldx) in dt, K values per row; out: (M, ldo) in
 * out_dt.  With fuse != 0 and 4 < M <= 32, N < 16384, kpad(K) <= 1920 the quantization runs inside
 * the product (one launch); otherwise, or with fuse == 0, the codes go through ws (same result bit
 * for bit).  ws: tesm_hip_bitlinear_fwd_ws_bytes(M, K) bytes. */
int64_t tesm_hip_bitlinear_fwd_ws_bytes(int64_t M, int64_t K);
int tesm_hip_bitlinear_fwd(const void* x, int dt, int64_t ldx, float eps, const uint8_t* packed, int64_t ldw,
                           const float* c_w, int c_w_per_row, const void* bias, int64_t M, int64_t N, int64_t K,
                           void* out, int out_dt, int64_t ldo, int fuse, void* ws, int64_t ws_bytes, void* stream);

/* State scan h_t = d_t h_{t-1} + u_t over (B, L, C), C contiguous.  Replaces
 * TESM_SISO._parallel_state_scan (tesm.py:1091-1164, torch branch; chunk_size = state_scan_chunk_size
 * reproduces its 1e-12 clamp semantics) and chunk_state_scan (ops/cuda/__init__.py:140-150).
 * decay/update: element (b,t,c) at ptr[(b*L+t)*ld + c], dt; states likewise in out_dt.
 * h0, h_final: (B, C) float64, nullable.  ws: tesm_hip_scan_ws_bytes() bytes, any contents (each call
 * clears what it uses); with ws 8-byte aligned and chunk_size <= 32 the scan is one pass (decoupled
 * look-back across workgroups), otherwise three passes.  Calls that share a workspace must be ordered
 * (same stream). */
int64_t tesm_hip_scan_ws_bytes(int64_t B, int64_t L, int64_t C, int64_t chunk_size);
int tesm_hip_scan(const void* decay, int64_t ld_decay, const void* update, int64_t ld_update, int dt, int64_t B,
                  int64_t L, int64_t C, int64_t chunk_size, const double* h0, void* states, int64_t ld_states,
                  int out_dt, double* h_final, void* ws, int64_t ws_bytes, void* stream);

/* RoPE cos/sin table for positions pos_offset..pos_offset+L-1: tab[t*(R/2)+i] = (cos, sin) of
 * pos * (1 / base**(2i/R)), rounded to dt.  Replaces the table built inside TESM_SISO._apply_rope
 * (tesm.py:783-793).  tab: (L, R/2) float2 (8 bytes each). */
int tesm_hip_rope_table(void* tab, int64_t L, int64_t R, int64_t pos_offset, double base, int dt, void* stream);

/* Causal local-window ternary entanglement + mix.  Replaces TESM_SISO._compute_local_entanglement
 * (tesm.py:853-952, torch branch) and the mix of TESM_SISO.forward (tesm.py:1231-1232, 1256), and
 * (mimo = 1) TESMMIMO_Optimized._compute_local_entanglement_mimo (tesm_mimo.py:394-588).
 * q, k: raw (pre-RoPE) queries/keys, element (b,t,h,r) at ptr[(b*L+t)*ld + h*R + r]; rope: table of
 * tesm_hip_rope_table for positions 0..L-1; q_add: optional cross-layer query bias added after
 * RoPE; bias: (H, W) float32 holding dt-rounded values; thr: threshold rounded to dt.
 * S: states, element (b,t,h,d) at S[(b*L+t)*ld_s + h*D + d].  Outputs (each nullable) share ld_out:
 * avg (window average), e_out (E = S + scale*(avg - S)), c_out (E - S), e_tanh (tanh E).
 * tern: optional int8 ternary map (B, L, H, W_eff).  ws: tesm_hip_local_ent_ws_bytes() bytes. */
int64_t tesm_hip_local_ent_ws_bytes(int64_t B, int64_t L, int64_t H, int64_t W);
int tesm_hip_local_ent(const void* q, int64_t ld_q, const void* k, int64_t ld_k, const void* rope, const void* q_add,
                       int64_t ld_qadd, const float* bias, const void* S, int64_t ld_s, int dt, int mimo, int64_t B,
                       int64_t L, int64_t H, int64_t R, int64_t D, int64_t W, float thr, float ent_scale, void* avg,
                       void* e_out, void* c_out, void* e_tanh, int64_t ld_out, int8_t* tern, void* ws,
                       int64_t ws_bytes, void* stream);

/* Local-window entanglement fused with the per-token int8 quantization of its two consumers'
 * inputs: tanh(E) (state_proj) and C = E - S (ent_proj).  Replaces, in one kernel,
 * TESM_SISO._compute_local_entanglement (tesm.py:853-952), the mix (tesm.py:1231-1232, 1256) and
 * BitLinear.quantized_input of state_proj / ent_proj (tesm.py:206-209).  SISO only, d_state <= 512.
 * Operand conventions as tesm_hip_local_ent (H = 1); codes are layout 1 with row stride ldq >=
 * kpad(D).  e_tanh / c_out (ld_out) optionally receive the float values as well. */
typedef struct tesm_hip_ent_quant {
  int dt;
  int64_t B, L, R, D, W;
  float thr, ent_scale, eps;
  const void* q;
  int64_t ld_q;
  const void* k;
  int64_t ld_k;
  const void* rope;
  const void* q_add;
  int64_t ld_qadd;
  const float* bias;          /* (W) float32 holding dt values */
  const void* S;
  int64_t ld_s;
  int8_t* q_te;
  float* s_te;
  int32_t* rs_te;
  int8_t* q_c;
  float* s_c;
  int32_t* rs_c;
  int64_t ldq;
  void* e_tanh;               /* optional */
  void* c_out;                /* optional */
  int64_t ld_out;
  int8_t* tern;               /* optional (B, L, min(W, L)) ternary map */
} tesm_hip_ent_quant;

int tesm_hip_local_ent_quant(const tesm_hip_ent_quant* p, void* stream);

/* One packed BitLinear as the fused layer drivers consume it. */
typedef struct tesm_hip_linear {
  const uint8_t* packed; /* (N, ldw) */
  int64_t ldw;
  const float* c_w;      /* device scalar (or (N) if c_w_per_row) */
  int c_w_per_row;
} tesm_hip_linear;

/* Output gate y = local + sigmoid(gate) * state_proj(tanh E) + ent_proj(E - S) from the codes of
 * tanh(E) and C.  Replaces tesm.py:1256-1260 (state_proj/ent_proj BitLinears and the gate) and,
 * when q_y is given, BitLinear.quantized_input of out_proj (tesm.py:206-209): the kernel then owns
 * whole rows (d_model <= 1024) and writes y's layout-1 codes (and y itself only if y != NULL).
 * local / gate: raw in_proj slices (dt), element (m, n) at ptr[m*ld + n]. */
typedef struct tesm_hip_output_gate {
  int dt;
  int64_t M, d_model, d_state;
  float eps;
  const int8_t* q_te;
  int64_t ldq_te;
  const float* s_te;
  const int32_t* rs_te;
  const int8_t* q_c;
  int64_t ldq_c;
  const float* s_c;
  const int32_t* rs_c;
  tesm_hip_linear state_proj, ent_proj;
  const void* local;
  int64_t ld_local;
  const void* gate;
  int64_t ld_gate;
  void* y;                    /* (M, ld_y) in dt; required when q_y is NULL */
  int64_t ld_y;
  int8_t* q_y;                /* optional (M, ldq_y) codes for out_proj */
  int64_t ldq_y;
  float* s_y;
  int32_t* rs_y;
} tesm_hip_output_gate;

int tesm_hip_output_gate_i2(const tesm_hip_output_gate* p, void* stream);

/* Whole TESM_SISO prefill forward (eval, no grad).  Replaces TESM_SISO.forward
 * (tesm.py:1175-1272): in_proj, gates, RoPE, cross-layer query bias, state scan, local (window > 0)
 * or global (window == 0) entanglement, mix, state_proj/ent_proj with the output gate
 * y = local + sigmoid(gate) * state_proj(tanh E) + ent_proj(E - S), out_proj.  With k_cache and
 * v_cache set it also fills the decode ring buffers as the reference's prefill does
 * (tesm.py:1235-1253): the last n = min(L, window) RoPE'd keys and states go to slots
 * window - n .. window - 1 (the caller sets cache_idx = 0, seq_pos = L, state = h_final). */
typedef struct tesm_hip_siso_layer {
  int dt;                     /* activations / module dtype */
  int64_t B, L, d_model, d_state, ent_rank, window, chunk_size;
  float bit_eps, thr, ent_scale;
  const void* u;              /* (B, L, d_model), contiguous */
  tesm_hip_linear in_proj, state_proj, ent_proj, out_proj, cross_q_proj;
  const void* decay_bias;     /* (d_state) in dt */
  const float* local_bias;    /* (window) float32 holding dt values */
  const void* rope;           /* tesm_hip_rope_table(L, ent_rank, 0) */
  const void* cross_state;    /* optional (B, L, d_state) in dt (previous layer's states) */
  const double* h0;           /* optional (B, d_state) */
  void* y;                    /* (B, L, d_model) */
  void* states;               /* (B, L, d_state) in dt */
  double* h_final;            /* optional (B, d_state) */
  void* proj_out;             /* optional (B, L, N_in) copy target; NULL = workspace only */
  void* k_cache;              /* optional (B, cache_window, ent_rank) ring of keys, cache_dt */
  void* v_cache;              /* optional (B, cache_window, d_state) ring of states, cache_dt */
  int cache_dt;               /* 0 f32, 1 bf16 */
  /* window == 0: global causal entanglement (tesm.py:963-1063) with the relative-position bias
   * parameters global_rel_pos_embed (global_dim), _scale (1), _bias (1), float32 holding dt values */
  const float* global_embed;
  int64_t global_dim;
  const float* global_scale;
  const float* global_bias;
  int64_t cache_window;       /* ring size of k_cache / v_cache (0: window) */
} tesm_hip_siso_layer;

int64_t tesm_hip_siso_prefill_ws_bytes(const tesm_hip_siso_layer* p);
int tesm_hip_siso_prefill(const tesm_hip_siso_layer* p, void* ws, int64_t ws_bytes, void* stream);

/* One TESM_SISO decode step for B sequences (one token each).  Replaces
 * TESM_SISO._forward_incremental (tesm.py:1274-1400) on the cache of allocate_inference_cache
 * (tesm.py:620-670): in_proj, gates, RoPE at position seq_pos, cross-layer query, the float64
 * state update new = decay * state + write * tanh(sv), ring write of (key, new) at slot cache_idx,
 * window scores over the ring in the reference's read order, strict ternary, count
 * normalisation, mix, the output gate and out_proj.  The caller then advances the host
 * bookkeeping: cache_idx = (cache_idx + 1) % window, seq_pos += 1. */
typedef struct tesm_hip_siso_step {
  int dt;                     /* module dtype */
  int cache_dt;               /* ring buffer dtype: 0 f32, 1 bf16 */
  int64_t B, d_model, d_state, ent_rank, window;
  int64_t seq_pos;            /* tokens seen before this one (its RoPE position) */
  int64_t cache_idx;          /* ring slot this step writes */
  float bit_eps, thr, ent_scale;
  const void* u;              /* (B, d_model) in dt */
  tesm_hip_linear in_proj, state_proj, ent_proj, out_proj, cross_q_proj;
  const void* decay_bias;     /* (d_state) in dt */
  const float* local_bias;    /* (window) float32 holding dt values */
  const void* rope;           /* tesm_hip_rope_table with at least seq_pos + 1 rows from position 0 */
  const void* cross_state;    /* optional (B, d_state) in dt */
  const double* state;        /* (B, d_state) float64 state before the step */
  double* state_out;          /* (B, d_state) float64 state after the step (may equal state) */
  void* k_cache;              /* (B, window, ent_rank) cache_dt, updated in place */
  void* v_cache;              /* (B, window, d_state) cache_dt, updated in place */
  void* y;                    /* (B, d_model) in dt */
  void* new_state;            /* optional (B, d_state) in dt: this step's state */
  int64_t ld_u;               /* row pitch of u in elements (0: d_model) */
  /* optional device int64[2] = {seq_pos, cache_idx}.  When set, the step reads its position and ring
   * slot there at run time (the host fields above are not used) and advances them at its end
   * ({seq_pos + 1, (cache_idx + 1) % window}), so one captured HIP graph of this call serves every
   * following step.  rope must then hold rope_rows >= every position the graph reaches (positions
   * past it read the last row). */
  int64_t* step_pos;
  int64_t rope_rows;
} tesm_hip_siso_step;

int64_t tesm_hip_siso_decode_ws_bytes(const tesm_hip_siso_step* p);
int tesm_hip_siso_decode(const tesm_hip_siso_step* p, void* ws, int64_t ws_bytes, void* stream);

/* The same decode step with no workspace argument and no allocation anywhere: the step's scratch
 * (activation codes, the in_proj output, the gate output) lives in a fixed array of
 * TESM_HIP_NOALLOC_SCRATCH_BYTES per device inside the library, held until the process ends.  No
 * reference counterpart: it is for callers that cannot allocate (code under HIP graph capture,
 * serving loops that forbid allocation).  A step whose tesm_hip_siso_decode_ws_bytes exceeds the
 * array is refused (TESM_ERR_WORKSPACE).  Every call on one device shares that device's array:
 * calls that overlap on one device (different streams, or threads) race and must be serialised by
 * the caller.  Results are bit-identical to tesm_hip_siso_decode. */
#define TESM_HIP_NOALLOC_SCRATCH_BYTES (8 << 20)
int tesm_hip_siso_decode_noalloc(const tesm_hip_siso_step* p, void* stream);

/* MIMO rank merge factors.  TESMMIMO_Optimized expands each head's update into mimo_rank copies
 * scaled by mimo_x and merges the entangled copies with mimo_o (tesm_mimo.py:963-1017); the scan
 * and the window mix are linear in the update and the window weights do not depend on the rank,
 * so the merge is the per-channel factor coef[h,d] = sum_r mimo_x[h,r,d]^2 * mimo_o[h,r,d] and the
 * rank-0 states are x0sq[h,d] = mimo_x[h,0,d]^2 times the rank-free ones.  mimo_x, mimo_o:
 * (n_heads, mimo_rank, d_state) in dt; coef, x0sq: (n_heads, d_state) float32. */
int tesm_hip_mimo_coef(const void* mimo_x, const void* mimo_o, int dt, int64_t n_heads, int64_t mimo_rank,
                       int64_t d_state, float* coef, float* x0sq, void* stream);

/* Whole TESMMIMO_Optimized prefill forward (eval, no grad).  Replaces TESMMIMO_Optimized.forward
 * (tesm_mimo.py:914-1062) with the ranks collapsed (tesm_hip_mimo_coef): in_proj, per-head gates,
 * one float32 state scan over n_heads * d_state channels (tesm_mimo.py:375-392), RoPE, the
 * per-head window entanglement with the reference's early-window truncation (tesm_mimo.py:525-588),
 * the rank merge, state_proj(tanh) / ent_proj with the output gate, out_proj.  With k_cache and
 * v_cache set it fills the decode ring buffers with the last min(L, window) RoPE'd keys and rank-0
 * states (tesm_mimo.py:1022-1037). */
typedef struct tesm_hip_mimo_layer {
  int dt;                     /* activations / module dtype */
  int64_t B, L, d_model, d_state, n_heads, ent_rank, window;
  float bit_eps, thr, ent_scale;
  const void* u;              /* (B, L, d_model), contiguous */
  tesm_hip_linear in_proj, state_proj, ent_proj, out_proj;
  const void* decay_bias;     /* (n_heads, d_state) in dt */
  const float* local_bias;    /* (n_heads, window) float32 holding dt values */
  const void* rope;           /* tesm_hip_rope_table(L, ent_rank, 0) */
  const float* mimo_coef;     /* (n_heads, d_state) from tesm_hip_mimo_coef */
  const float* mimo_x0sq;     /* (n_heads, d_state) from tesm_hip_mimo_coef */
  void* y;                    /* (B, L, d_model) */
  double* h_final;            /* optional (B, n_heads, d_state): rank-0 state after the last token */
  float* last_state;          /* optional (B, n_heads, d_state): the same in float32 */
  void* k_cache;              /* optional (B, window, n_heads, ent_rank), cache_dt */
  void* v_cache;              /* optional (B, window, n_heads, d_state), cache_dt */
  int cache_dt;               /* 0 f32, 1 bf16 */
  /* optional entanglement statistics (tesm_mimo.py:458-523, window branch): hard ternary of
   * q.k/sqrt(ent_rank) over the first S = min(L, 64) positions' complete windows of W = min(window, L)
   * slots, (B, S-W+1, n_heads, W) in dt, and per batch row (#positive, #negative, #zero) */
  void* stats_ternary;
  int32_t* stats_counts;      /* (B, 3) */
  /* window == 0: global causal entanglement over the flattened heads (tesm_mimo.py:590-687) */
  const float* global_embed;
  int64_t global_dim;
  const float* global_scale;
  const float* global_bias;
  int64_t cache_window;       /* ring size of k_cache / v_cache (0: window) */
} tesm_hip_mimo_layer;

int64_t tesm_hip_mimo_prefill_ws_bytes(const tesm_hip_mimo_layer* p);
int tesm_hip_mimo_prefill(const tesm_hip_mimo_layer* p, void* ws, int64_t ws_bytes, void* stream);

/* One TESMMIMO_Optimized decode step for B sequences (one token each).  Replaces
 * TESMMIMO_Optimized._forward_incremental (tesm_mimo.py:753-912) on the cache of
 * allocate_inference_cache (tesm_mimo.py:689-731): in_proj, per-head gates, RoPE at position
 * seq_pos, the optional cross-layer query cross_q_proj(cross_state) per head (a (B, n_heads, d_state)
 * state, tesm_mimo.py:818-826), the float64 per-head state update (no rank expansion, as the
 * reference's step), ring write of (key, state) at slot cache_idx, per-head window scores with the
 * head's bias row, strict ternary, count normalisation, mix, then state_proj(tanh(E)) and ent_proj(C)
 * over the flattened heads, the output gate and out_proj.  The caller then advances
 * cache_idx = (cache_idx + 1) % window and seq_pos += 1.  window 1 with a zero bias is the
 * global-entanglement layer's step (its rings hold one slot). */
typedef struct tesm_hip_mimo_step {
  int dt;                     /* module dtype */
  int cache_dt;               /* ring buffer dtype: 0 f32, 1 bf16 */
  int64_t B, d_model, d_state, n_heads, ent_rank, window;
  int64_t seq_pos;            /* tokens seen before this one (its RoPE position) */
  int64_t cache_idx;          /* ring slot this step writes */
  float bit_eps, thr, ent_scale;
  const void* u;              /* (B, d_model) in dt, row pitch ld_u */
  int64_t ld_u;               /* row pitch of u in elements (0: d_model) */
  tesm_hip_linear in_proj, state_proj, ent_proj, out_proj, cross_q_proj;
  const void* decay_bias;     /* (n_heads, d_state) in dt */
  const float* local_bias;    /* (n_heads, window) float32 holding dt values */
  const void* rope;           /* tesm_hip_rope_table with at least seq_pos + 1 rows from position 0 */
  const void* cross_state;    /* optional (B, n_heads, d_state) in dt */
  const double* state;        /* (B, n_heads, d_state) float64 state before the step */
  double* state_out;          /* (B, n_heads, d_state) float64 state after the step (may equal state) */
  void* k_cache;              /* (B, window, n_heads, ent_rank) cache_dt, updated in place */
  void* v_cache;              /* (B, window, n_heads, d_state) cache_dt, updated in place */
  void* y;                    /* (B, d_model) in dt */
  void* new_state;            /* optional (B, n_heads, d_state) in dt: this step's state */
} tesm_hip_mimo_step;

int64_t tesm_hip_mimo_decode_ws_bytes(const tesm_hip_mimo_step* p);
int tesm_hip_mimo_decode(const tesm_hip_mimo_step* p, void* ws, int64_t ws_bytes, void* stream);

/* Residual add + RMSNorm of the TESM block (block.py:7-17, 27-31 and 38-41): with `residual` set,
 * s = x + residual in the promoted dtype (float32 when either is float32); `residual_out` (may alias
 * `residual`) receives s in residual_out_dt (float32 for residual_in_fp32); then
 * y = RMSNorm(s.to(dt)) = x * rsqrt(mean(x^2) + eps) * weight, every op rounded to dt.  With `q` set
 * the kernel also writes y's per-token int8 codes (tesm.py:206-209) in the product layout, as
 * tesm_hip_quant_act_i8(layout 1) would, for a BitLinear that reads y; `y` itself is then optional.
 * D <= 16384. */
typedef struct tesm_hip_rmsnorm {
  int dt;                     /* module dtype: x, weight, y */
  int64_t M, D;
  float eps;
  const void* x;              /* (M, ld_x) */
  int64_t ld_x;
  const void* residual;       /* optional (M, ld_res) in residual_dt */
  int residual_dt;
  int64_t ld_res;
  void* residual_out;         /* optional (M, ld_res_out) in residual_out_dt */
  int residual_out_dt;
  int64_t ld_res_out;
  const void* weight;         /* (D) in dt */
  void* y;                    /* optional (M, ld_y) in dt */
  int64_t ld_y;
  int8_t* q;                  /* optional (M, ldq) int8 codes of y, ldq >= tesm_hip_kpad(D) */
  int64_t ldq;
  float* s_x;                 /* (M) code scales (with q) */
  int32_t* rowsum;            /* (M) code sums (with q) */
  float bit_eps;
} tesm_hip_rmsnorm;

int tesm_hip_add_rmsnorm(const tesm_hip_rmsnorm* p, void* stream);

/* FeedForward of the TESM block (mixer_seq_simple.py:25-67, eval): gate and up share the per-token
 * int8 codes of x (the reference's grouped projection, :45-57: one quantized input against the
 * concatenated gate / up weights, each with its own absmean scale); one pass computes both products
 * and h = silu(gate) * up in the module dtype's op order; h is quantized per token and down_proj
 * gives y.  x is either given in dt or as layout-1 codes (x_codes, x_scale, x_rowsum, e.g. from
 * tesm_hip_add_rmsnorm). */
typedef struct tesm_hip_ffn {
  int dt;
  int64_t M, d_model, d_inter;
  float bit_eps;
  const void* x;              /* (M, ld_x) in dt, or NULL with x_codes */
  int64_t ld_x;
  const int8_t* x_codes;      /* optional (M, ldq_x) layout-1 codes of x, ldq_x >= tesm_hip_kpad(d_model) */
  int64_t ldq_x;
  const float* x_scale;       /* (M) */
  const int32_t* x_rowsum;    /* (M) */
  tesm_hip_linear gate_proj, up_proj, down_proj;
  void* y;                    /* (M, ld_y) in dt */
  int64_t ld_y;
} tesm_hip_ffn;

int64_t tesm_hip_ffn_ws_bytes(const tesm_hip_ffn* p);
int tesm_hip_ffn_forward(const tesm_hip_ffn* p, void* ws, int64_t ws_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TESM_HIP_H_ */
