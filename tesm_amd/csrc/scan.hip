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
// Three launches, all channel-parallel (lanes along C, coalesced):
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
    } else {
      const float sv = rnd<DT>(tanhf_(ld<DT>(a.sv, tok * a.ld_sv + ch)));
      d = rnd<DT>(sigmoidf_(rnd<DT>(ld<DT>(a.decay, tok * a.ld_decay + ch) + ld<DT>(a.decay_bias, ch))));
      const float w = rnd<DT>(sigmoidf_(ld<DT>(a.update, tok * a.ld_update + ch)));
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
    if constexpr (MODE == 1) Vec<DT, CPT>::load(a.sv, tok * a.ld_sv + ch, x2[i]);
  }
  float d[TM][CPT], u[TM][CPT];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
      if constexpr (MODE == 0) {
        d[i][j] = x0[i][j];
        u[i][j] = x1[i][j];
      } else {
        const float sv = rnd<DT>(tanhf_(x2[i][j]));
        d[i][j] = rnd<DT>(sigmoidf_(rnd<DT>(x0[i][j] + bias[j])));
        const float w = rnd<DT>(sigmoidf_(x1[i][j]));
        u[i][j] = a.round_update ? rnd<DT>(w * sv) : w * sv;
      }
      if (i >= n) {
        d[i][j] = 1.0f;
        u[i][j] = 0.0f;
      }
    }
  }
  if constexpr (MODE == 1 && PHASE == 1) {
    if (a.gated) {  // the gated decay and update, for the apply pass (dt values, (B*L, C) each)
      const int64_t plane = a.B * a.L * a.C;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if (i >= n) continue;
        const int64_t o = (b * a.L + t0 + i) * a.C + ch;
        if constexpr (DT == kBF16 && CPT == 2) {
          *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.gated) + o) = pack_bf16x2(d[i][0], d[i][1]);
          *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(a.gated) + plane + o) = pack_bf16x2(u[i][0], u[i][1]);
        } else {
#pragma unroll
          for (int j = 0; j < CPT; ++j) {
            st<DT>(a.gated, o + j, d[i][j]);
            st<DT>(a.gated, plane + o + j, u[i][j]);
          }
        }
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

template <int DT, int OUT_DT, int MODE, int TM, int CPT>
int run_scan_fast(const ScanArgs& a, int64_t T, int64_t nc, float* summ, float* carry, hipStream_t st) {
  const int64_t threads = a.B * nc * (a.C / CPT);
  const unsigned nb = static_cast<unsigned>((threads + 255) / 256);
  // the gate pass is VALU-heavy: one channel per thread for twice the waves
  constexpr int CPT1 = MODE == 1 ? 1 : CPT;
  const unsigned nb1 = static_cast<unsigned>((a.B * nc * (a.C / CPT1) + 255) / 256);
  scan_fast_kernel<DT, OUT_DT, MODE, 1, TM, CPT1><<<nb1, 256, 0, st>>>(a, T, nc, summ, carry);
  dim3 g2(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(a.B));
  if (nc >= 64)
    scan_carry_seg_kernel<16><<<g2, 16 * 64, 0, st>>>(a, nc, summ, carry);
  else
    scan_carry_seg_kernel<4><<<g2, 4 * 64, 0, st>>>(a, nc, summ, carry);
  if (MODE == 1 && a.gated) {
    // apply pass on the stored gates: a plain decay / update scan
    ScanArgs g = a;
    g.mode = 0;
    g.decay = a.gated;
    g.ld_decay = a.C;
    g.update = static_cast<const char*>(a.gated) + a.B * a.L * a.C * (DT == kBF16 ? 2 : 4);
    g.ld_update = a.C;
    scan_fast_kernel<DT, OUT_DT, 0, 3, TM, CPT><<<nb, 256, 0, st>>>(g, T, nc, summ, carry);
  } else {
    scan_fast_kernel<DT, OUT_DT, MODE, 3, TM, CPT><<<nb, 256, 0, st>>>(a, T, nc, summ, carry);
  }
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
  scan_chunk_kernel<DT, OUT_DT, MODE, 1><<<g3, 64, 0, st>>>(a, T, nc, summ, carry);
  dim3 g2(static_cast<unsigned>((a.C + 63) / 64), static_cast<unsigned>(a.B));
  scan_carry_kernel<<<g2, 64, 0, st>>>(a, nc, summ, carry);
  scan_chunk_kernel<DT, OUT_DT, MODE, 3><<<g3, 64, 0, st>>>(a, T, nc, summ, carry);
  return check_launch("scan");
}

}  // namespace

// Thread-chunk length: a multiple of the reference chunk (so the clamp's running product restarts
// inside a thread) of at most 16 positions when possible.
int64_t scan_chunk_len(int64_t L, int64_t cs) {
  const int64_t cse = std::max<int64_t>(1, std::min(cs, L));
  return cse >= 16 ? cse : cse * (16 / cse);
}

int64_t scan_ws_bytes(int64_t B, int64_t L, int64_t C, int64_t cs) {
  if (L <= 0) return 0;
  const int64_t T = scan_chunk_len(L, cs);
  const int64_t nc = (L + T - 1) / T;
  return round_up(B * nc * C * 3 * static_cast<int64_t>(sizeof(float)), 256);
}

int launch_scan(const ScanArgs& a, void* ws, int64_t ws_bytes, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "scan: input dtype must be 0 or 1");
  TESM_REQUIRE(a.out_dt == kF32 || a.out_dt == kBF16, kErrInvalidArg, "scan: output dtype must be 0 or 1");
  TESM_REQUIRE(a.mode == 0 || a.mode == 1, kErrInvalidArg, "scan: mode must be 0 (decay/update) or 1 (gates)");
  TESM_REQUIRE(a.B >= 0 && a.L >= 0 && a.C >= 1 && a.cs >= 1, kErrInvalidArg, "scan: bad sizes");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.decay && a.update && a.states, kErrInvalidArg, "scan: null pointer");
  TESM_REQUIRE(a.ld_decay >= a.C && a.ld_update >= a.C && a.ld_states >= a.C, kErrInvalidArg, "scan: ld < C");
  if (a.mode == 1)
    TESM_REQUIRE(a.sv && a.decay_bias && a.ld_sv >= a.C, kErrInvalidArg, "scan mode 1: need sv and decay_bias");
  TESM_REQUIRE(!a.gated || (a.mode == 1 && a.round_update && a.out_dt == a.dt), kErrInvalidArg,
               "scan: a gate buffer needs mode 1 with rounded updates");
  const int64_t need = scan_ws_bytes(a.B, a.L, a.C, a.cs);
  TESM_REQUIRE(ws && ws_bytes >= need, kErrWorkspace, "scan: workspace too small");
  const int64_t T = scan_chunk_len(a.L, a.cs);
  const int64_t nc = (a.L + T - 1) / T;
  TESM_REQUIRE(nc <= 65535 && a.B <= 65535, kErrUnsupported, "scan: too many chunks or batch rows");
  float* summ = static_cast<float*>(ws);
  float* carry = summ + 2 * a.B * nc * a.C;
  // the reference chunk grid starts at 0 with chunk = min(cs, L); pass the effective value
  ScanArgs e = a;
  e.cs = std::max<int64_t>(1, std::min(a.cs, a.L));
  const bool pairs = a.dt == kBF16 && a.C % 2 == 0 && a.ld_decay % 2 == 0 && a.ld_update % 2 == 0 &&
                     (a.mode == 0 || a.ld_sv % 2 == 0) && a.ld_states % 2 == 0 && aligned(a.decay, 4) &&
                     aligned(a.update, 4) && (a.mode == 0 || (aligned(a.sv, 4) && aligned(a.decay_bias, 4))) &&
                     aligned(a.states, 4) && (!a.gated || aligned(a.gated, 4));
  if (T <= 32) {
    if (a.dt == kBF16) {
      if (a.out_dt == kBF16) {
        if (a.mode == 0) return scan_fast_dispatch<kBF16, kBF16, 0>(e, T, nc, summ, carry, pairs, st);
        return scan_fast_dispatch<kBF16, kBF16, 1>(e, T, nc, summ, carry, pairs, st);
      }
      if (a.mode == 0) return scan_fast_dispatch<kBF16, kF32, 0>(e, T, nc, summ, carry, pairs, st);
      return scan_fast_dispatch<kBF16, kF32, 1>(e, T, nc, summ, carry, pairs, st);
    }
    if (a.out_dt == kF32) {
      if (a.mode == 0) return scan_fast_dispatch<kF32, kF32, 0>(e, T, nc, summ, carry, false, st);
      return scan_fast_dispatch<kF32, kF32, 1>(e, T, nc, summ, carry, false, st);
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
    default: return fail(kErrInvalidArg, "scan: unsupported dtype combination");
  }
}

}  // namespace tesm
