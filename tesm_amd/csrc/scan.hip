// Chunked parallel state scan for gfx950:  h_t = d_t * h_{t-1} + g_t * u_t  over (B, L, C).
//
// Reference (torch branch): tesm_ssm/modules/tesm.py:1065-1164 (SISO) and
// tesm_ssm/modules/tesm_mimo.py:375-392 (MIMO, sequential, no clamps).
// The SISO reference evaluates each chunk of `state_scan_chunk_size` positions in closed form,
//   A = cumprod(max(d, 1e-12)),  s = A * (h0 + cumsum(u / max(A, 1e-12))),
// which is the recurrence above with g_t = A_t / max(A_t, 1e-12) (A_t = product of the clamped
// decays since the start of the reference chunk).  g_t = 1 except when a within-chunk product
// falls below 1e-12; the kernels reproduce that factor ("clamp" mode) and run the recurrence in
// fp32 registers.
//
// Default: one pass with decoupled look-back across workgroups (scan_lb_kernel, below), which reads
// the inputs once.  Fallback (chunks longer than 32 positions, or a workspace that is not 8-byte
// aligned): three launches, all channel-parallel (lanes along C, coalesced):
//   1. summary: each (b, chunk of T positions, channel) scans its chunk from h = 0 and stores
//      (prod d, h_end);
//   2. carry:   each (b, channel) folds the chunk summaries in order -> carry into every chunk
//      and the final state (fp64 at the API);
//   3. apply:   each (b, chunk, channel) rescans its chunk from its carry and writes the states.
// Gate fusion ("mode 1") reads the raw in_proj slices and evaluates
//   d = sigmoid(decay_raw + decay_bias), u = sigmoid(write_raw) * tanh(sv_raw)
// with the reference's rounding points (tesm.py:1202-1205, 1222).
#include "tesm_hip_internal.h"
#include "scan.h"

namespace tesm {

namespace {

constexpr float kScanEps = 1e-12f;
constexpr float kScanInvEps = 1e12f;  // the clamp factor A / 1e-12 as a product

template <int DT, int MODE>
struct ScanIn {
  const ScanArgs& a;
  __device__ __forceinline__ void at(int64_t b, int64_t t, int64_t ch, float& d, float& u) const {
    const int64_t tok = b * a.L + t;
    if constexpr (MODE == 0) {
      d = ld<DT>(a.decay, tok * a.ld_decay + ch);
      u = ld<DT>(a.update, tok * a.ld_update + ch);
    } else if constexpr (MODE == 1) {
      const float sv = rnd<DT>(tanhf_(ld<DT>(a.sv, tok * a.ld_sv + ch)));
      d = rnd<DT>(sigmoidf_(rnd<DT>(ld<DT>(a.decay, tok * a.ld_decay + ch) + ld<DT>(a.decay_bias, ch))));
      const float w = rnd<DT>(sigmoidf_(ld<DT>(a.update, tok * a.ld_update + ch)));
      u = a.round_update ? rnd<DT>(w * sv) : w * sv;
    } else {  // gates applied by the producer
      const float sv = ld<DT>(a.sv, tok * a.ld_sv + ch);
      d = ld<DT>(a.decay, tok * a.ld_decay + ch);
      const float w = ld<DT>(a.update, tok * a.ld_update + ch);
      u = a.round_update ? rnd<DT>(w * sv) : w * sv;
    }
  }
};

// PHASE 1: write chunk summary; PHASE 3: rescan from the carry and store states.
template <int DT, int OUT_DT, int MODE, int PHASE>
__global__ __launch_bounds__(64) void scan_chunk_kernel(ScanArgs a, int64_t T, int64_t nc, float* __restrict__ summ,
                                                        const float* __restrict__ carry) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  const int64_t c = blockIdx.y, b = blockIdx.z;
  if (ch >= a.C) return;
  const ScanIn<DT, MODE> in{a};
  const int64_t t0 = c * T, t1 = (t0 + T < a.L) ? t0 + T : a.L;
  const int64_t sidx = (b * nc + c) * a.C + ch;
  float h = (PHASE == 1) ? 0.0f : carry[sidx];
  float P = 1.0f, A = 1.0f;
  for (int64_t t = t0; t < t1; ++t) {
    float d, u;
    in.at(b, t, ch, d, u);
    float g = 1.0f;
    if (a.clamp) {
      d = fmaxf(d, kScanEps);
      A = ((t % a.cs) == 0) ? d : A * d;
      if (A < kScanEps) g = A * kScanInvEps;
    }
    h = d * h + g * u;
    if (PHASE == 1) {
      P *= d;
    } else {
      st<OUT_DT>(a.states, (b * a.L + t) * a.ld_states + ch, h);
    }
  }
  if (PHASE == 1) {
    summ[2 * sidx] = P;
    summ[2 * sidx + 1] = h;
  }
}

__global__ __launch_bounds__(64) void scan_carry_kernel(ScanArgs a, int64_t nc, const float* __restrict__ summ,
                                                        float* __restrict__ carry) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
  const int64_t b = blockIdx.y;
  if (ch >= a.C) return;
  float h = a.h0 ? static_cast<float>(a.h0[b * a.C + ch]) : 0.0f;
  for (int64_t c = 0; c < nc; ++c) {
    const int64_t sidx = (b * nc + c) * a.C + ch;
    carry[sidx] = h;
    h = summ[2 * sidx] * h + summ[2 * sidx + 1];
  }
  if (a.h_final) a.h_final[b * a.C + ch] = static_cast<double>(h);
}

// ---------------------------------------------------------------------------
// Fast path: TM positions per thread-chunk fully unrolled (all loads issued before the
// recurrence), CPT adjacent channels per thread (bf16 pairs -> 4-byte loads and stores).
// ---------------------------------------------------------------------------
template <int DT, int CPT>
struct Vec;
template <>
struct Vec<kBF16, 2> {
  __device__ static __forceinline__ void load(const void* p, int64_t i, float (&v)[2]) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p) + i);
    v[0] = __uint_as_float(w << 16);
    v[1] = __uint_as_float(w & 0xffff0000u);
  }
};
template <int DT>
struct Vec<DT, 1> {
  __device__ static __forceinline__ void load(const void* p, int64_t i, float (&v)[1]) { v[0] = ld<DT>(p, i); }
};

template <int DT, int OUT_DT, int MODE, int PHASE, int TM, int CPT>
__global__ __launch_bounds__(256) void scan_fast_kernel(ScanArgs a, int64_t T, int64_t nc, float* __restrict__ summ,
                                                        const float* __restrict__ carry) {
  const int64_t ng = a.C / CPT;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= a.B * nc * ng) return;
  const int64_t gq = idx % ng, rest = idx / ng;
  const int64_t c = rest % nc, b = rest / nc;
  const int64_t ch = gq * CPT;
  const int64_t t0 = c * T;
  const int n = static_cast<int>((t0 + T < a.L ? t0 + T : a.L) - t0);

  // All loads are issued unconditionally (positions past the end re-read the last valid one and
  // are masked afterwards) so that the whole chunk's loads are in flight at once.
  float x0[TM][CPT], x1[TM][CPT], x2[TM][CPT], bias[CPT];
  if constexpr (MODE == 1) Vec<DT, CPT>::load(a.decay_bias, ch, bias);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t tok = b * a.L + t0 + (i < n ? i : n - 1);
    Vec<DT, CPT>::load(a.decay, tok * a.ld_decay + ch, x0[i]);
    Vec<DT, CPT>::load(a.update, tok * a.ld_update + ch, x1[i]);
    if constexpr (MODE >= 1) Vec<DT, CPT>::load(a.sv, tok * a.ld_sv + ch, x2[i]);
  }
  float d[TM][CPT], u[TM][CPT];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      if constexpr (MODE == 0) {
        d[i][j] = x0[i][j];
        u[i][j] = x1[i][j];
      } else if constexpr (MODE == 1) {
        const float sv = rnd<DT>(tanhf_(x2[i][j]));
        d[i][j] = rnd<DT>(sigmoidf_(rnd<DT>(x0[i][j] + bias[j])));
        const float w = rnd<DT>(sigmoidf_(x1[i][j]));
        u[i][j] = a.round_update ? rnd<DT>(w * sv) : w * sv;
      } else {
        d[i][j] = x0[i][j];
        u[i][j] = a.round_update ? rnd<DT>(x1[i][j] * x2[i][j]) : x1[i][j] * x2[i][j];
      }
      if (i >= n) {
        d[i][j] = 1.0f;
        u[i][j] = 0.0f;
      }
    }
  }
  const int64_t sidx = (b * nc + c) * a.C + ch;
  const int cs = static_cast<int>(a.cs);  // the thread-chunk start is a multiple of cs
  float h[CPT], P[CPT], A[CPT];
#pragma unroll
  for (int j = 0; j < CPT; ++j) {
    h[j] = (PHASE == 1) ? 0.0f : carry[sidx + j];
    P[j] = 1.0f;
    A[j] = 1.0f;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    if (i < n) {
      const bool reset = (i % cs) == 0;
      float out[CPT];
#pragma unroll
      for (int j = 0; j < CPT; ++j) {
        float dd = d[i][j], g = 1.0f;
        if (a.clamp) {
          dd = fmaxf(dd, kScanEps);
          A[j] = reset ? dd : A[j] * dd;
          if (A[j] < kScanEps) g = A[j] * kScanInvEps;
        }
        h[j] = dd * h[j] + g * u[i][j];
        P[j] *= dd;
        out[j] = h[j];
      }
      if (PHASE == 3) {
        const int64_t o = (b * a.L + t0 + i) * a.ld_states + ch;
        if constexpr (OUT_DT == kBF16 && CPT == 2) {
          const uint32_t w = pack_bf16x2(out[0], out[1]);
          *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.states) + o) = w;
        } else {
#pragma unroll
          for (int j = 0; j < CPT; ++j) st<OUT_DT>(a.states, o + j, out[j]);
        }
      }
    }
  }
  if (PHASE == 1) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      summ[2 * (sidx + j)] = P[j];
      summ[2 * (sidx + j) + 1] = h[j];
    }
  }
}

// Carry propagation over the chunk summaries: a workgroup per (batch row, 64 channels) with
// NSEG waves, each folding a contiguous run of chunks; the runs are combined through LDS.
template <int NSEG>
__global__ __launch_bounds__(NSEG * 64) void scan_carry_seg_kernel(ScanArgs a, int64_t nc,
                                                                   const float* __restrict__ summ,
                                                                   float* __restrict__ carry) {
  __shared__ float segP[NSEG][64], segH[NSEG][64];
  const int lane = threadIdx.x & 63, seg = threadIdx.x >> 6;
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const int64_t b = blockIdx.y;
  const bool ok = ch < a.C;
  const int64_t per = (nc + NSEG - 1) / NSEG;
  const int64_t c0 = seg * per, c1 = (c0 + per < nc) ? c0 + per : nc;
  float Ps = 1.0f, Hs = 0.0f;
  if (ok) {
    for (int64_t c = c0; c < c1; ++c) {
      const int64_t sidx = (b * nc + c) * a.C + ch;
      const float P = summ[2 * sidx], H = summ[2 * sidx + 1];
      Hs = P * Hs + H;
      Ps *= P;
    }
  }
  segP[seg][lane] = Ps;
  segH[seg][lane] = Hs;
  __syncthreads();
  if (!ok) return;
  float h = a.h0 ? static_cast<float>(a.h0[b * a.C + ch]) : 0.0f;
  for (int s2 = 0; s2 < seg; ++s2) h = segP[s2][lane] * h + segH[s2][lane];
  for (int64_t c = c0; c < c1; ++c) {
    const int64_t sidx = (b * nc + c) * a.C + ch;
    carry[sidx] = h;
    h = summ[2 * sidx] * h + summ[2 * sidx + 1];
  }
  if (seg == NSEG - 1 && a.h_final) a.h_final[b * a.C + ch] = static_cast<double>(h);
}

// ---------------------------------------------------------------------------
// Single pass with decoupled look-back.  A tile is (batch row b, span c of SUB T positions, group g
// of 64 channels); its SUB waves (4 or 8) take one sub-span of T positions each (T is a multiple of the
// reference chunk, so the clamp's running product restarts inside a wave) and its lanes one channel
// each.  The workgroup index fixes the chain (b, g); the span c is the ticket the workgroup takes
// from its chain's counter when it starts, so every tile a tile waits on (earlier spans of its
// chain) took an earlier ticket and is already running; ticket 0 waits on nothing, so every wait
// ends.  One counter per chain, each on its own 256-byte line, keeps the ticket atomics from
// queueing on one cache line.
//
// A wave loads its sub-span and gates once and scans it from h = 0; the sub-span aggregates
// (prod d, h_end) meet in LDS, giving each wave the state entering its sub-span as a function of
// the tile's carry, and the tile's aggregate, which the tile publishes (flag 1).  It then finds
// its carry by looking back over earlier spans of the same (b, g), 64 at a time: wave 0 polls the
// flags, the nearest span whose end state is published (flag 2) ends the walk, and the aggregates
// in between are composed nearest first (an equal share of the window per wave, the shares
// combined through LDS).  Span 0 publishes its end state directly, so a walk never passes it.  The tile
// publishes its own end state (flag 2) and every wave rescans its sub-span from registers, writing
// the states.  A reset kernel clears the flags and the ticket before each pass.
//
// Cross-workgroup visibility without cache maintenance: the published values and the flags are
// written and read only with agent-scope atomic accesses (coherent at agent scope, across the XCDs'
// L2s, without the whole-L2 write-back and invalidate an agent-scope release / acquire costs).  A
// writer waits for its value stores to complete (s_waitcnt) before the workgroup barrier after which
// one thread stores the flag; a reader polls flags in one wave, and the other waves read values
// only after the barrier that follows.  A poll gives up after kScanSpinLimit rounds, so the launch
// completes whatever happens: the tile's states are then NaN and bit 0 of the device status word
// g_scan_status is set (tesm_hip_device_status reads and clears it).
// ---------------------------------------------------------------------------
constexpr int kScanLbCh = 64;    // channels per tile (one per lane)
// sub-spans per tile (one per wave): 4, or 8 for long chains (fewer spans to chain; with few spans
// per chain the shorter tile keeps more workgroups in flight)
constexpr int kScanSpinLimit = 1 << 20;

// Device status word of the look-back scan (one per device): bit 0 = a poll gave up.
__device__ unsigned g_scan_status;
// Poll limit of the next launches; a negative value makes every look-back give up at once, which
// tests use to exercise the failure report (tesm_hip_debug_scan_spin_limit).
int g_scan_spin_limit = kScanSpinLimit;

struct ScanLb {
  float2* agg;       // (B, nc, C): (prod d, h_end from 0) of every span
  float* incl;       // (B, nc, C): state at the end of every span
  int* flags;        // (B, nc, G): 0 nothing yet, 1 aggregate published, 2 end state published
  unsigned* ticket;  // span counter of chain x at ticket[x * kScanLbTicketStride]
  int spin_limit;    // poll rounds before giving up (< 0: give up without polling)
};
constexpr int kScanLbTicketStride = 64;  // ints: one 256-byte line per counter

// Clears the flags (n ints) and the chain counters (nt, strided) that follow them.
__global__ __launch_bounds__(256) void scan_lb_reset_kernel(int* p, int64_t n, int64_t nt) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
  else if (i < n + nt) p[n + (i - n) * kScanLbTicketStride] = 0;
}

__device__ __forceinline__ int scan_flag_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void scan_flag_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void scan_agg_store(float2* p, float x, float y) {
  const unsigned long long v = (static_cast<unsigned long long>(__float_as_uint(y)) << 32) | __float_as_uint(x);
  __hip_atomic_store(reinterpret_cast<unsigned long long*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 scan_agg_load(const float2* p) {
  const unsigned long long v = __hip_atomic_load(reinterpret_cast<const unsigned long long*>(p), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float(static_cast<unsigned>(v)), __uint_as_float(static_cast<unsigned>(v >> 32)));
}
__device__ __forceinline__ void scan_val_store(float* p, float x) {
  __hip_atomic_store(p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float scan_val_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Streaming (non-temporal) gate loads and state stores of the activated-gate mode: the MIMO scan
// reads its gates once and writes float32 states that are read back only after the whole scan
// (configs[4]: 1.6 GB and 1.07 GB), so caching either only evicts other lines.
template <int DT>
__device__ __forceinline__ float ld_stream(const void* p, int64_t i) {
  if constexpr (DT == kBF16) {
    const uint32_t h = __builtin_nontemporal_load(static_cast<const uint16_t*>(p) + i);
    return __uint_as_float(h << 16);
  } else {
    return __builtin_nontemporal_load(static_cast<const float*>(p) + i);
  }
}
template <int MODE, int OUT_DT>
__device__ __forceinline__ void st_state(void* p, int64_t i, float v) {
  if constexpr (MODE == 2 && OUT_DT == kF32)
    __builtin_nontemporal_store(v, static_cast<float*>(p) + i);
  else
    st<OUT_DT>(p, i, v);
}

// CR: the clamp / update-rounding semantics, 1 = both (SISO), 0 = neither (MIMO), 2 = read from a.
template <int DT, int OUT_DT, int MODE, int TM, int SUB, int CR>
__global__ __launch_bounds__(kScanLbCh * SUB) void scan_lb_kernel(ScanArgs a, int64_t T, int64_t nc, int64_t G,
                                                                  ScanLb s) {
  const bool clamp = CR == 2 ? a.clamp != 0 : CR == 1;
  const bool round_update = CR == 2 ? a.round_update != 0 : CR == 1;
  constexpr int WIN = 64 / SUB;  // look-back window entries composed per wave
  __shared__ unsigned s_tile;
  __shared__ int s_m, s_stop;
  __shared__ float2 s_sub[SUB][kScanLbCh];  // sub-span aggregates, then window shares
  // the wave index is uniform: read it into a scalar register so that position offsets are scalar math
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t chain = blockIdx.x % (a.B * G);  // grid = nc workgroups per chain
  if (tid == 0) s_tile = atomicAdd(&s.ticket[chain * kScanLbTicketStride], 1u);
  __syncthreads();
  const int64_t c = s_tile;
  const int64_t b = chain / G, g = chain % G;
  const int64_t ch = g * kScanLbCh + lane;
  const bool on = ch < a.C;
  const int64_t chc = on ? ch : a.C - 1;  // idle lanes read a valid channel and store nothing
  const int64_t t0 = (c * SUB + w) * T;  // this wave's first position
  const int n = t0 >= a.L ? 0 : static_cast<int>(t0 + T < a.L ? T : a.L - t0);  // wave-uniform

  // 1. the sub-span's inputs and gates (all loads in flight at once; positions past the end re-read
  //    the last one and become d = 1, u = 0), then its scan from h = 0
  float d[TM], u[TM];
  float h = 0.0f, P = 1.0f;
  if (n > 0) {
    float x0[TM], x1[TM], x2[TM], bias = 0.0f;
    if constexpr (MODE == 1) bias = ld<DT>(a.decay_bias, chc);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t tok = b * a.L + t0 + (i < n ? i : n - 1);
      if constexpr (MODE == 2) {
        x0[i] = ld_stream<DT>(a.decay, tok * a.ld_decay + chc);
        x1[i] = ld_stream<DT>(a.update, tok * a.ld_update + chc);
        x2[i] = ld_stream<DT>(a.sv, tok * a.ld_sv + chc);
      } else {
        x0[i] = ld<DT>(a.decay, tok * a.ld_decay + chc);
        x1[i] = ld<DT>(a.update, tok * a.ld_update + chc);
        if constexpr (MODE == 1) x2[i] = ld<DT>(a.sv, tok * a.ld_sv + chc);
      }
    }
    const int cs = static_cast<int>(a.cs);
    float A = 1.0f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      float dd, uu;
      if constexpr (MODE == 0) {
        dd = x0[i];
        uu = x1[i];
      } else if constexpr (MODE == 1) {
        const float sv = rnd<DT>(tanhf_(x2[i]));
        dd = rnd<DT>(sigmoidf_(rnd<DT>(x0[i] + bias)));
        const float wr = rnd<DT>(sigmoidf_(x1[i]));
        uu = round_update ? rnd<DT>(wr * sv) : wr * sv;
      } else {
        dd = x0[i];
        uu = round_update ? rnd<DT>(x1[i] * x2[i]) : x1[i] * x2[i];
      }
      if (clamp) {
        dd = fmaxf(dd, kScanEps);
        A = (i % cs) == 0 ? dd : A * dd;
        if (A < kScanEps) uu *= A * kScanInvEps;  // the clamp factor, folded into the update
      }
      if (i >= n) {
        dd = 1.0f;
        uu = 0.0f;
      }
      d[i] = dd;
      u[i] = uu;
      h = dd * h + uu;
      P *= dd;
    }
  } else {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      d[i] = 1.0f;
      u[i] = 0.0f;
    }
  }

  // 2. sub-spans -> the state entering this wave's sub-span (pp * carry + ph) and the tile aggregate
  s_sub[w][lane] = make_float2(P, h);
  __syncthreads();
  float pp = 1.0f, ph = 0.0f, tp = 1.0f, th = 0.0f;
#pragma unroll
  for (int v = 0; v < SUB; ++v) {
    const float2 e = s_sub[v][lane];
    if (v == w) {
      pp = tp;
      ph = th;
    }
    th = e.x * th + e.y;
    tp *= e.x;
  }

  // 3. the tile's carry
  const int64_t fb = b * nc * G + g;      // flag of span k: fb + k * G
  const int64_t vb = b * nc * a.C + chc;  // values of span k: vb + k * C
  float carry;
  if (c == 0) {
    carry = a.h0 ? static_cast<float>(a.h0[b * a.C + chc]) : 0.0f;
  } else {
    if (w == 0 && on) scan_agg_store(&s.agg[vb + c * a.C], tp, th);
    __builtin_amdgcn_s_waitcnt(0);  // the value stores are complete before the flag can be stored
    __syncthreads();                // (and every wave has read s_sub)
    if (tid == 0) scan_flag_store(&s.flags[fb + c * G], 1);
    float accP = 1.0f, accH = 0.0f;
    int64_t k0 = c - 1;  // nearest span not composed yet; k0 >= 0 (span 0 ends every walk)
    for (;;) {
      if (w == 0) {
        // lane l watches span k0 - l; lanes before span 0 never report
        const int64_t k = k0 - lane;
        int m = 0, stop = 2;
        for (int it = 0;; ++it) {
          if (s.spin_limit < 0) {
            m = 0;
            stop = 2;
            break;
          }
          const int f = k >= 0 ? scan_flag_load(&s.flags[fb + k * G]) : 0;
          const unsigned long long incl = __ballot(f == 2), ready = __ballot(f >= 1);
          if (incl) {
            m = __ffsll(static_cast<long long>(incl)) - 1;    // aggregates to compose before it
            const unsigned long long need = (2ull << m) - 1;  // lanes 0..m (all ones for m = 63)
            if ((ready & need) == need) {
              stop = 1;
              break;
            }
          } else if (ready == ~0ull) {  // 64 aggregates, no end state among them: compose, go on
            m = 64;
            stop = 0;
            break;
          }
          if (it >= s.spin_limit) {
            m = 0;
            stop = 2;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) {
          s_m = m;
          s_stop = stop;
        }
      }
      __syncthreads();
      const int m = s_m, stop = s_stop;
      // wave w composes window entries j0 .. j1 - 1 (spans k0 - j, all >= 0), nearest first
      const int j0 = w * WIN, j1 = m < j0 + WIN ? m : j0 + WIN;
      float qP = 1.0f, qH = 0.0f;
      if (j0 < j1) {
        float2 v[WIN];
#pragma unroll
        for (int j = 0; j < WIN; ++j) {
          const int jj = j0 + j < j1 ? j0 + j : j1 - 1;
          v[j] = scan_agg_load(&s.agg[vb + (k0 - jj) * a.C]);
        }
#pragma unroll
        for (int j = 0; j < WIN; ++j) {
          if (j0 + j < j1) {
            qH += qP * v[j].y;
            qP *= v[j].x;
          }
        }
      }
      s_sub[w][lane] = make_float2(qP, qH);
      __syncthreads();
#pragma unroll
      for (int q = 0; q < SUB; ++q) {
        const float2 e = s_sub[q][lane];
        accH += accP * e.y;
        accP *= e.x;
      }
      if (stop == 1) {
        carry = accH + accP * scan_val_load(&s.incl[vb + (k0 - m) * a.C]);
        break;
      }
      if (stop == 2) {  // gave up waiting: NaN states and the status bit report the failure
        carry = __builtin_nanf("");
        if (tid == 0) __hip_atomic_fetch_or(&g_scan_status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      k0 -= 64;
      __syncthreads();  // s_m, s_stop and s_sub are rewritten by the next round
    }
  }
  const float hend = tp * carry + th;
  if (c < nc - 1) {  // publish the end state for later spans
    if (w == 0 && on) scan_val_store(&s.incl[vb + c * a.C], hend);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) scan_flag_store(&s.flags[fb + c * G], 2);
  } else if (w == 0 && on && a.h_final) {
    a.h_final[b * a.C + ch] = static_cast<double>(hend);
  }

  // 4. rescan the sub-span from its entering state and store the states
  if (!on || n <= 0) return;
  float hh = pp * carry + ph;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    if (i < n) {
      hh = d[i] * hh + u[i];
      st_state<MODE, OUT_DT>(a.states, (b * a.L + t0 + i) * a.ld_states + ch, hh);
    }
  }
}

// Look-back launch geometry for thread-chunk length T: spans of sub * T positions, groups of
// kScanLbCh channels.
struct ScanLbShape {
  int64_t nc, G, tiles;
  int sub;
};
ScanLbShape scan_lb_shape(int64_t B, int64_t L, int64_t C, int64_t T) {
  ScanLbShape g;
  g.sub = (L + 4 * T - 1) / (4 * T) > 16 ? 8 : 4;
  g.nc = (L + g.sub * T - 1) / (g.sub * T);
  g.G = (C + kScanLbCh - 1) / kScanLbCh;
  g.tiles = B * g.nc * g.G;
  return g;
}

template <int DT, int OUT_DT, int MODE, int CR>
int run_scan_lb_cr(const ScanArgs& a, int64_t T, float* summ, int* flags, hipStream_t st) {
  const ScanLbShape sh = scan_lb_shape(a.B, a.L, a.C, T);
  ScanLb s;
  s.agg = reinterpret_cast<float2*>(summ);
  s.incl = summ + 2 * a.B * sh.nc * a.C;
  s.flags = flags;
  s.ticket = reinterpret_cast<unsigned*>(flags + sh.tiles);
  s.spin_limit = __atomic_load_n(&g_scan_spin_limit, __ATOMIC_RELAXED);
  const int64_t nchain = a.B * sh.G;
  if (!a.flags_clear)
    scan_lb_reset_kernel<<<static_cast<unsigned>((sh.tiles + nchain + 255) / 256), 256, 0, TESM_LOGGED(st, scan_lb_reset_kernel)>>>(flags, sh.tiles,
                                                                                                 nchain);
  const unsigned grid = static_cast<unsigned>(sh.tiles);
  if (sh.sub == 8) {
    if (T <= 16)
      scan_lb_kernel<DT, OUT_DT, MODE, 16, 8, CR><<<grid, kScanLbCh * 8, 0, TESM_LOGGED(st, scan_lb_kernel<DT, OUT_DT, MODE, 16, 8, CR>)>>>(a, T, sh.nc, sh.G, s);
    else
      scan_lb_kernel<DT, OUT_DT, MODE, 32, 8, CR><<<grid, kScanLbCh * 8, 0, TESM_LOGGED(st, scan_lb_kernel<DT, OUT_DT, MODE, 32, 8, CR>)>>>(a, T, sh.nc, sh.G, s);
  } else {
    if (T <= 16)
      scan_lb_kernel<DT, OUT_DT, MODE, 16, 4, CR><<<grid, kScanLbCh * 4, 0, TESM_LOGGED(st, scan_lb_kernel<DT, OUT_DT, MODE, 16, 4, CR>)>>>(a, T, sh.nc, sh.G, s);
    else
      scan_lb_kernel<DT, OUT_DT, MODE, 32, 4, CR><<<grid, kScanLbCh * 4, 0, TESM_LOGGED(st, scan_lb_kernel<DT, OUT_DT, MODE, 32, 4, CR>)>>>(a, T, sh.nc, sh.G, s);
  }
  return check_launch("scan look-back");
}

// Gate modes fix the clamp / rounding semantics at compile time (both or neither); the
// decay / update mode reads them.
template <int DT, int OUT_DT, int MODE>
int run_scan_lb(const ScanArgs& a, int64_t T, float* summ, int* flags, hipStream_t st) {
  if constexpr (MODE >= 1) {
    if (a.clamp) return run_scan_lb_cr<DT, OUT_DT, MODE, 1>(a, T, summ, flags, st);
    return run_scan_lb_cr<DT, OUT_DT, MODE, 0>(a, T, summ, flags, st);
  } else {
    return run_scan_lb_cr<DT, OUT_DT, MODE, 2>(a, T, summ, flags, st);
  }
}

template <int DT, int OUT_DT, int MODE, int TM, int CPT>
int run_scan_fast(const ScanArgs& a, int64_t T, int64_t nc, float* summ, float* carry, hipStream_t st) {
  const int64_t threads = a.B * nc * (a.C / CPT);
  const unsigned nb = static_cast<unsigned>((threads + 255) / 256);
  // the gate pass is VALU-heavy: one channel per thread for twice the waves
  constexpr int CPT1 = MODE == 1 ? 1 : CPT;
  const unsigned nb1 = static_cast<unsigned>((a.B * nc * (a.C / CPT1) + 255) / 256);
  scan_fast_kernel<DT, OUT_DT, MODE, 1, TM, CPT1><<<nb1, 256, 0, TESM_LOGGED(st, scan_fast_kernel<DT, OUT_DT, MODE, 1, TM, CPT1>)>>>(a, T, nc, summ, carry);
  dim3 g2(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(a.B));
  if (nc >= 64)
    scan_carry_seg_kernel<16><<<g2, 16 * 64, 0, TESM_LOGGED(st, scan_carry_seg_kernel<16>)>>>(a, nc, summ, carry);
  else
    scan_carry_seg_kernel<4><<<g2, 4 * 64, 0, TESM_LOGGED(st, scan_carry_seg_kernel<4>)>>>(a, nc, summ, carry);
  scan_fast_kernel<DT, OUT_DT, MODE, 3, TM, CPT><<<nb, 256, 0, TESM_LOGGED(st, scan_fast_kernel<DT, OUT_DT, MODE, 3, TM, CPT>)>>>(a, T, nc, summ, carry);
  return check_launch("scan");
}

template <int DT, int OUT_DT, int MODE>
int scan_fast_dispatch(const ScanArgs& e, int64_t T, int64_t nc, float* summ, float* carry, bool pairs,
                       hipStream_t st) {
  if constexpr (DT == kBF16) {
    if (pairs)
      return T <= 16 ? run_scan_fast<DT, OUT_DT, MODE, 16, 2>(e, T, nc, summ, carry, st)
                     : run_scan_fast<DT, OUT_DT, MODE, 32, 2>(e, T, nc, summ, carry, st);
  }
  return T <= 16 ? run_scan_fast<DT, OUT_DT, MODE, 16, 1>(e, T, nc, summ, carry, st)
                 : run_scan_fast<DT, OUT_DT, MODE, 32, 1>(e, T, nc, summ, carry, st);
}

template <int DT, int OUT_DT, int MODE>
int run_scan(const ScanArgs& a, int64_t T, int64_t nc, float* summ, float* carry, hipStream_t st) {
  dim3 g3(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(nc), static_cast<unsigned>(a.B));
  scan_chunk_kernel<DT, OUT_DT, MODE, 1><<<g3, 64, 0, TESM_LOGGED(st, scan_chunk_kernel<DT, OUT_DT, MODE, 1>)>>>(a, T, nc, summ, carry);
  dim3 g2(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(a.B));
  scan_carry_kernel<<<g2, 64, 0, TESM_LOGGED(st, scan_carry_kernel)>>>(a, nc, summ, carry);
  scan_chunk_kernel<DT, OUT_DT, MODE, 3><<<g3, 64, 0, TESM_LOGGED(st, scan_chunk_kernel<DT, OUT_DT, MODE, 3>)>>>(a, T, nc, summ, carry);
  return check_launch("scan");
}

}  // namespace

// Thread-chunk length: a multiple of the reference chunk (so the clamp's running product restarts
// inside a thread) of at most 16 positions when possible.
int64_t scan_chunk_len(int64_t L, int64_t cs) {
  const int64_t cse = std::max<int64_t>(1, std::min(cs, L));
  return cse >= 16 ? cse : cse * (16 / cse);
}

namespace {
bool scan_lb_eligible(int64_t B, int64_t L, int64_t C, int64_t T, const void* ws) {
  return T <= 32 && aligned(ws, 8) && scan_lb_shape(B, L, C, T).tiles < (1 << 23);
}
// the flag region follows the chunk summaries and carries (nc = chunks of the thread-chunk length)
int* scan_lb_flags(int64_t B, int64_t C, int64_t nc, void* ws) {
  return reinterpret_cast<int*>(static_cast<char*>(ws) + round_up(B * nc * C * 3 * static_cast<int64_t>(sizeof(float)), 256));
}
}  // namespace

void scan_lb_clear_range(int64_t B, int64_t L, int64_t C, int64_t cs, void* ws, int** p, int64_t* n) {
  *p = nullptr;
  *n = 0;
  if (B <= 0 || L <= 0 || C <= 0 || !ws) return;
  const int64_t T = scan_chunk_len(L, cs);
  if (!scan_lb_eligible(B, L, C, T, ws)) return;
  const ScanLbShape sh = scan_lb_shape(B, L, C, T);
  *p = scan_lb_flags(B, C, (L + T - 1) / T, ws);
  *n = sh.tiles + B * sh.G * kScanLbTicketStride;  // flags, then the strided chain counters
}

int64_t scan_ws_bytes(int64_t B, int64_t L, int64_t C, int64_t cs) {
  if (L <= 0) return 0;
  const int64_t T = scan_chunk_len(L, cs);
  const int64_t nc = (L + T - 1) / T;
  const int64_t G = (C + kScanLbCh - 1) / kScanLbCh;
  // chunk summaries and carries (3 floats per (b, chunk, channel); the look-back pass's spans are
  // longer than chunks, so its aggregates and end states fit too), then the look-back flags per
  // (b, span, channel group) (at most one span per chunk) and a span counter per (b, channel group),
  // one 256-byte line each
  return round_up(B * nc * C * 3 * static_cast<int64_t>(sizeof(float)), 256) +
         round_up((B * nc * G + B * G * kScanLbTicketStride) * static_cast<int64_t>(sizeof(int)), 256);
}

int launch_scan(const ScanArgs& a, void* ws, int64_t ws_bytes, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "scan: input dtype must be 0 or 1");
  TESM_REQUIRE(a.out_dt == kF32 || a.out_dt == kBF16, kErrInvalidArg, "scan: output dtype must be 0 or 1");
  TESM_REQUIRE(a.mode >= 0 && a.mode <= 2, kErrInvalidArg,
               "scan: mode must be 0 (decay/update), 1 (gates) or 2 (activated gates)");
  TESM_REQUIRE(a.B >= 0 && a.L >= 0 && a.C >= 1 && a.cs >= 1, kErrInvalidArg, "scan: bad sizes");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.decay && a.update && a.states, kErrInvalidArg, "scan: null pointer");
  TESM_REQUIRE(a.ld_decay >= a.C && a.ld_update >= a.C && a.ld_states >= a.C, kErrInvalidArg, "scan: ld < C");
  if (a.mode >= 1) {
    TESM_REQUIRE(a.sv && (a.decay_bias || a.mode == 2) && a.ld_sv >= a.C, kErrInvalidArg,
                 "scan gate modes: need sv (and decay_bias in mode 1)");
    TESM_REQUIRE((a.clamp != 0) == (a.round_update != 0), kErrUnsupported,
                 "scan gate modes: clamp and round_update must agree (SISO: both, MIMO: neither)");
  }
  const int64_t need = scan_ws_bytes(a.B, a.L, a.C, a.cs);
  TESM_REQUIRE(ws && ws_bytes >= need, kErrWorkspace, "scan: workspace too small");
  const int64_t T = scan_chunk_len(a.L, a.cs);
  const int64_t nc = (a.L + T - 1) / T;
  TESM_REQUIRE(nc <= 65535 && a.B <= 65535, kErrUnsupported, "scan: too many chunks or batch rows");
  float* summ = static_cast<float*>(ws);
  float* carry = summ + 2 * a.B * nc * a.C;
  int* flags = scan_lb_flags(a.B, a.C, nc, ws);
  // the reference chunk grid starts at 0 with chunk = min(cs, L); pass the effective value
  ScanArgs e = a;
  e.cs = std::max<int64_t>(1, std::min(a.cs, a.L));
  const bool pairs = a.dt == kBF16 && a.C % 2 == 0 && a.ld_decay % 2 == 0 && a.ld_update % 2 == 0 &&
                     (a.mode == 0 || a.ld_sv % 2 == 0) && a.ld_states % 2 == 0 && aligned(a.decay, 4) &&
                     aligned(a.update, 4) && (a.mode == 0 || aligned(a.sv, 4)) &&
                     (a.mode != 1 || aligned(a.decay_bias, 4)) && aligned(a.states, 4);
  if (scan_lb_eligible(a.B, a.L, a.C, T, ws)) {
    // single pass with decoupled look-back
    const int key = a.dt * 100 + a.out_dt * 10 + a.mode;
    switch (key) {
      case 0: return run_scan_lb<kF32, kF32, 0>(e, T, summ, flags, st);
      case 1: return run_scan_lb<kF32, kF32, 1>(e, T, summ, flags, st);
      case 110: return run_scan_lb<kBF16, kBF16, 0>(e, T, summ, flags, st);
      case 111: return run_scan_lb<kBF16, kBF16, 1>(e, T, summ, flags, st);
      case 100: return run_scan_lb<kBF16, kF32, 0>(e, T, summ, flags, st);
      case 101: return run_scan_lb<kBF16, kF32, 1>(e, T, summ, flags, st);
      case 10: return run_scan_lb<kF32, kBF16, 0>(e, T, summ, flags, st);
      case 11: return run_scan_lb<kF32, kBF16, 1>(e, T, summ, flags, st);
      case 2: return run_scan_lb<kF32, kF32, 2>(e, T, summ, flags, st);
      case 112: return run_scan_lb<kBF16, kBF16, 2>(e, T, summ, flags, st);
      case 102: return run_scan_lb<kBF16, kF32, 2>(e, T, summ, flags, st);
      case 12: return run_scan_lb<kF32, kBF16, 2>(e, T, summ, flags, st);
      default: return fail(kErrInvalidArg, "scan: unsupported dtype combination");
    }
  }
  if (T <= 32) {
    if (a.dt == kBF16) {
      if (a.out_dt == kBF16) {
        if (a.mode == 0) return scan_fast_dispatch<kBF16, kBF16, 0>(e, T, nc, summ, carry, pairs, st);
        if (a.mode == 1) return scan_fast_dispatch<kBF16, kBF16, 1>(e, T, nc, summ, carry, pairs, st);
        return scan_fast_dispatch<kBF16, kBF16, 2>(e, T, nc, summ, carry, pairs, st);
      }
      if (a.mode == 0) return scan_fast_dispatch<kBF16, kF32, 0>(e, T, nc, summ, carry, pairs, st);
      if (a.mode == 1) return scan_fast_dispatch<kBF16, kF32, 1>(e, T, nc, summ, carry, pairs, st);
      return scan_fast_dispatch<kBF16, kF32, 2>(e, T, nc, summ, carry, pairs, st);
    }
    if (a.out_dt == kF32) {
      if (a.mode == 0) return scan_fast_dispatch<kF32, kF32, 0>(e, T, nc, summ, carry, false, st);
      if (a.mode == 1) return scan_fast_dispatch<kF32, kF32, 1>(e, T, nc, summ, carry, false, st);
      return scan_fast_dispatch<kF32, kF32, 2>(e, T, nc, summ, carry, false, st);
    }
  }
  const int key = a.dt * 100 + a.out_dt * 10 + a.mode;
  switch (key) {
    case 0: return run_scan<kF32, kF32, 0>(e, T, nc, summ, carry, st);
    case 1: return run_scan<kF32, kF32, 1>(e, T, nc, summ, carry, st);
    case 110: return run_scan<kBF16, kBF16, 0>(e, T, nc, summ, carry, st);
    case 111: return run_scan<kBF16, kBF16, 1>(e, T, nc, summ, carry, st);
    case 100: return run_scan<kBF16, kF32, 0>(e, T, nc, summ, carry, st);
    case 101: return run_scan<kBF16, kF32, 1>(e, T, nc, summ, carry, st);
    case 10: return run_scan<kF32, kBF16, 0>(e, T, nc, summ, carry, st);
    case 11: return run_scan<kF32, kBF16, 1>(e, T, nc, summ, carry, st);
    case 2: return run_scan<kF32, kF32, 2>(e, T, nc, summ, carry, st);
    case 112: return run_scan<kBF16, kBF16, 2>(e, T, nc, summ, carry, st);
    case 102: return run_scan<kBF16, kF32, 2>(e, T, nc, summ, carry, st);
    case 12: return run_scan<kF32, kBF16, 2>(e, T, nc, summ, carry, st);
    default: return fail(kErrInvalidArg, "scan: unsupported dtype combination");
  }
}

int scan_status(unsigned* out, int clear) {
  unsigned v = 0;
  hipError_t e = hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_scan_status), sizeof(v), 0, hipMemcpyDeviceToHost);
  if (e == hipSuccess && clear && v != 0) {
    const unsigned zero = 0;
    e = hipMemcpyToSymbol(HIP_SYMBOL(g_scan_status), &zero, sizeof(zero), 0, hipMemcpyHostToDevice);
  }
  if (e != hipSuccess) return fail(kErrLaunch, std::string("device status: ") + hipGetErrorString(e));
  if (out) *out = v;
  return kOk;
}

void scan_set_spin_limit(int limit) { __atomic_store_n(&g_scan_spin_limit, limit, __ATOMIC_RELAXED); }

}  // namespace tesm
