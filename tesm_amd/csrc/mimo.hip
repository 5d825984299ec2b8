// TESMMIMO_Optimized (tesm_ssm/modules/tesm_mimo.py:914-1062) around the shared kernels.
//
// The reference expands every head's update into mimo_rank copies, scans each copy and runs the
// window entanglement on each, then merges with mimo_o.  Decay and window weights are shared by the
// ranks and the scan and the window mix are linear in the update, so
//   states_r = S * mimo_x[:, r]^2,  sum_r entangled_r * mimo_o[:, r] = E * c,  c = sum_r mimo_x_r^2 mimo_o_r,
// with S the scan of write * tanh(sv) and E its entangled state.  Here the one scan and the one mix
// run on S and the merge is a per-channel factor (float32 throughout, as the reference's rank tensors).
#include "mimo.h"

namespace tesm {

namespace {

template <int DT>
__global__ __launch_bounds__(256) void mimo_coef_kernel(const void* x, const void* o, int64_t H, int64_t Rm, int64_t D,
                                                        float* coef, float* x0sq) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= H * D) return;
  const int64_t h = i / D, d = i - h * D;
  float c = 0.0f;
  for (int64_t r = 0; r < Rm; ++r) {
    const int64_t k = (h * Rm + r) * D + d;
    const float xv = ld<DT>(x, k);
    c += (xv * xv) * ld<DT>(o, k);
  }
  const float x0 = ld<DT>(x, h * Rm * D + d);
  coef[i] = c;
  x0sq[i] = x0 * x0;
}

constexpr int kMixTP = 64;           // positions per workgroup
constexpr int kMixDS = 32;           // channels per block
constexpr int kMixSP = kMixDS + 8;   // state row pitch (floats): rows r and r + 4 fall in opposite bank halves
constexpr int kMixWP = kMixTP + 4;   // weight row pitch (floats)
constexpr int kMixCB = 16;           // channel blocks per workgroup
constexpr int kMixLD = 4;            // float4 state loads per thread per block: (kMixTP + 63) * 8 <= 4 * 256

// Window mix for one (batch row, head) pair, kMixTP positions x kMixCB blocks of kMixDS channels.
// Key position of window slot w is t - W + 1 + w (tesm_mimo.py:536-586); slots the reference drops
// carry weight 0.  The weights (transposed, [w][position]) are staged in LDS once; the states of one
// channel block plus its W - 1 row halo are staged per block, and the next block's states are loaded
// into registers while the current one is mixed and stored.  Each thread owns 2 positions x 4 channels
// and walks the window keeping the 2 state rows it needs in registers, so every 8 multiply-adds cost
// one state and one weight read.  Sums run over w in increasing order.  WT is W when it is a
// compile-time case (index math by shifts), else 0.
template <int DT, bool VEC, int WT>
__global__ __launch_bounds__(256) void mimo_mix_kernel(MimoMixArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_mimo[];
  const int W = WT > 0 ? WT : static_cast<int>(a.W);
  const int rows = kMixTP + W - 1;
  float* srow = lds_mimo;                  // [rows][kMixSP]
  float* wtT = lds_mimo + rows * kMixSP;   // [W][kMixWP]
  const int64_t bh = blockIdx.z;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kMixTP;
  const int64_t nblk = (a.D + kMixDS - 1) / kMixDS;
  const int64_t cb0 = static_cast<int64_t>(blockIdx.x) * kMixCB;
  const int64_t cb1 = cb0 + kMixCB < nblk ? cb0 + kMixCB : nblk;
  const int tid = threadIdx.x;
  const int64_t C = a.H * a.D;
  const int64_t tlo = t0 - (W - 1);  // position of LDS row 0
  const int nvalid = static_cast<int>(a.L - t0 < kMixTP ? a.L - t0 : kMixTP);
  const float* Sh = a.S + (b * a.L) * C + h * a.D;

  // state prefetch of channel block cb into registers (rows outside [0, L) and channels past D are 0)
  float4 pre[kMixLD];
  auto prefetch = [&](int64_t cb) {
#pragma unroll
    for (int k = 0; k < kMixLD; ++k) {
      const int i = tid + k * 256;
      const int r = i >> 3, c4 = 4 * (i & 7);
      const int64_t t = tlo + r;
      const int64_t dc = cb * kMixDS + c4;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (r < rows && t >= 0 && t < a.L) {
        const float* src = Sh + t * C + dc;
        if (VEC && dc + 3 < a.D) {
          v = *reinterpret_cast<const float4*>(src);
        } else {
          if (dc + 0 < a.D) v.x = src[0];
          if (dc + 1 < a.D) v.y = src[1];
          if (dc + 2 < a.D) v.z = src[2];
          if (dc + 3 < a.D) v.w = src[3];
        }
      }
      pre[k] = v;
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int k = 0; k < kMixLD; ++k) {
      const int i = tid + k * 256;
      const int r = i >> 3, c4 = 4 * (i & 7);
      if (r < rows) *reinterpret_cast<float4*>(srow + r * kMixSP + c4) = pre[k];
    }
  };
  prefetch(cb0);
  const float* wb = a.wts + ((b * a.L + t0) * a.H + h) * W;
  const int64_t wrow = a.H * W;  // floats between the weights of consecutive positions
  for (int i = tid; i < kMixTP * W; i += 256) {
    const int p = i / W, w = i - p * W;
    wtT[w * kMixWP + p] = p < nvalid ? wb[p * wrow + w] : 0.0f;
  }
  stage();
  __syncthreads();
  const int p0 = 2 * (tid >> 3), c0 = 4 * (tid & 7);
  const float* sp = srow + p0 * kMixSP + c0;
  for (int64_t cb = cb0; cb < cb1; ++cb) {
    prefetch(cb + 1 < cb1 ? cb + 1 : cb);  // the last block re-reads itself (never staged)
    float acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    float4 s0 = *reinterpret_cast<const float4*>(sp);
#pragma unroll 4
    for (int w = 0; w < W; ++w) {
      const float4 s1 = *reinterpret_cast<const float4*>(sp + (w + 1) * kMixSP);
      const float2 wv = *reinterpret_cast<const float2*>(wtT + w * kMixWP + p0);
      acc[0][0] = __builtin_fmaf(wv.x, s0.x, acc[0][0]);
      acc[0][1] = __builtin_fmaf(wv.x, s0.y, acc[0][1]);
      acc[0][2] = __builtin_fmaf(wv.x, s0.z, acc[0][2]);
      acc[0][3] = __builtin_fmaf(wv.x, s0.w, acc[0][3]);
      acc[1][0] = __builtin_fmaf(wv.y, s1.x, acc[1][0]);
      acc[1][1] = __builtin_fmaf(wv.y, s1.y, acc[1][1]);
      acc[1][2] = __builtin_fmaf(wv.y, s1.z, acc[1][2]);
      acc[1][3] = __builtin_fmaf(wv.y, s1.w, acc[1][3]);
      s0 = s1;
    }
    const int64_t d = cb * kMixDS + c0;
    float cf[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) cf[j] = d + j < a.D ? a.coef[h * a.D + d + j] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      if (p0 + i >= nvalid) break;
      const int64_t t = t0 + p0 + i;
      const float* srq = srow + (p0 + i + W - 1) * kMixSP + c0;  // the query position's own state
      float te[4], cc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float sv = srq[j];
        const float e = sv + a.ent_scale * (acc[i][j] - sv);
        te[j] = tanhf_(e * cf[j]);
        cc[j] = (e - sv) * cf[j];
      }
      const int64_t o = (b * a.L + t) * C + h * a.D + d;
      if (VEC && d + 3 < a.D) {
        st4<DT>(a.te, o, te);
        st4<DT>(a.cc, o, cc);
      } else {
        for (int j = 0; j < 4 && d + j < a.D; ++j) {
          st<DT>(a.te, o + j, te[j]);
          st<DT>(a.cc, o + j, cc[j]);
        }
      }
    }
    __syncthreads();  // every thread is done with this block's states
    if (cb + 1 < cb1) {
      stage();
      __syncthreads();
    }
  }
}

__global__ __launch_bounds__(256) void mimo_final_kernel(const float* S, const float* x0sq, int64_t B, int64_t L,
                                                         int64_t C, double* h_final, float* last) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= B * C) return;
  const int64_t b = i / C, c = i - b * C;
  const float v = S[(b * L + L - 1) * C + c] * x0sq[c];
  if (h_final) h_final[i] = static_cast<double>(v);
  if (last) last[i] = v;
}

// One workgroup per batch row; one thread per (v, h, w) score, products summed in natural r order.
template <int DT>
__global__ __launch_bounds__(256) void mimo_stats_kernel(MimoStatsArgs a) {
  __shared__ int32_t cnt[3][4];
  const int64_t b = blockIdx.x;
  const int64_t half = a.R / 2;
  // window branch: (v, h, w) over V = S - W + 1 complete windows; global branch: (s, t) over S x S
  const int64_t V = a.global ? a.S : a.S - a.W + 1;
  const int64_t n = a.global ? a.S * a.S : V * a.H * a.W;
  int32_t pos = 0, neg = 0;
  for (int64_t e = threadIdx.x; e < n; e += 256) {
    int64_t tq, tk, h0, h1;
    if (a.global) {
      tq = e / a.S;
      tk = e % a.S;
      h0 = 0;
      h1 = a.H;
    } else {
      const int64_t v = e / (a.H * a.W), w = e % a.W;
      h0 = (e / a.W) % a.H;
      h1 = h0 + 1;
      tq = a.W - 1 + v;
      tk = v + w;
    }
    // products in natural (h, r) order: per head the first halves (r < R/2) then the second halves;
    // the loop is unrolled so a batch of loads is in flight before the running sum needs it
    float acc = 0.0f;
    for (int64_t h = h0; h < h1; ++h) {
      const int64_t qo = (b * a.L + tq) * a.ld_q + h * a.R, ko = (b * a.L + tk) * a.ld_k + h * a.R;
      for (int part = 0; part < 2; ++part) {
#pragma unroll 8
        for (int64_t i = 0; i < half; ++i) {
          float q1, q2, k1, k2;
          rope_pair<DT>(ld<DT>(a.q, qo + i), ld<DT>(a.q, qo + i + half), a.rope[tq * half + i], q1, q2);
          rope_pair<DT>(ld<DT>(a.k, ko + i), ld<DT>(a.k, ko + i + half), a.rope[tk * half + i], k1, k2);
          acc += part == 0 ? rnd<DT>(q1 * k1) : rnd<DT>(q2 * k2);
        }
      }
    }
    const float sc = rnd<DT>(rnd<DT>(acc) / a.sqrt_r);
    const float t = sc > a.thr ? 1.0f : (sc < -a.thr ? -1.0f : 0.0f);
    pos += t > 0.0f;
    neg += t < 0.0f;
    st<DT>(a.ternary, b * n + e, t);
  }
  // wave sums, then the workgroup's
  for (int o = 32; o > 0; o >>= 1) {
    pos += __shfl_xor(pos, o);
    neg += __shfl_xor(neg, o);
  }
  const int wv = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    cnt[0][wv] = pos;
    cnt[1][wv] = neg;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const int32_t p = cnt[0][0] + cnt[0][1] + cnt[0][2] + cnt[0][3];
    const int32_t q = cnt[1][0] + cnt[1][1] + cnt[1][2] + cnt[1][3];
    a.counts[b * 3 + 0] = p;
    a.counts[b * 3 + 1] = q;
    a.counts[b * 3 + 2] = static_cast<int32_t>(n) - p - q;
  }
}

}  // namespace

int launch_mimo_stats(const MimoStatsArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "mimo stats: dtype must be 0 or 1");
  if (a.B == 0) return kOk;
  TESM_REQUIRE(a.q && a.k && a.rope && a.ternary && a.counts, kErrInvalidArg, "mimo stats: null pointer");
  TESM_REQUIRE(a.global ? (a.S >= 1 && a.S <= a.L) : (a.W >= 1 && a.S >= a.W && a.S <= a.L), kErrInvalidArg,
               "mimo stats: need 1 <= W <= S <= L");
  TESM_REQUIRE(a.R >= 2 && a.R % 2 == 0 && a.H >= 1, kErrInvalidArg, "mimo stats: need an even R");
  TESM_REQUIRE((a.S - a.W + 1) * a.H * a.W <= 0x7fffffff, kErrUnsupported, "mimo stats: too many scores");
  if (a.dt == kBF16)
    mimo_stats_kernel<kBF16><<<static_cast<unsigned>(a.B), 256, 0, TESM_LOGGED(st, mimo_stats_kernel<kBF16>)>>>(a);
  else
    mimo_stats_kernel<kF32><<<static_cast<unsigned>(a.B), 256, 0, TESM_LOGGED(st, mimo_stats_kernel<kF32>)>>>(a);
  return check_launch("mimo stats");
}

int launch_mimo_coef(const void* mimo_x, const void* mimo_o, int dt, int64_t H, int64_t Rm, int64_t D, float* coef,
                     float* x0sq, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "mimo coef: dtype must be 0 or 1");
  TESM_REQUIRE(H >= 1 && Rm >= 1 && D >= 1, kErrInvalidArg, "mimo coef: bad sizes");
  TESM_REQUIRE(mimo_x && mimo_o && coef && x0sq, kErrInvalidArg, "mimo coef: null pointer");
  const unsigned nb = static_cast<unsigned>((H * D + 255) / 256);
  if (dt == kBF16)
    mimo_coef_kernel<kBF16><<<nb, 256, 0, TESM_LOGGED(st, mimo_coef_kernel<kBF16>)>>>(mimo_x, mimo_o, H, Rm, D, coef, x0sq);
  else
    mimo_coef_kernel<kF32><<<nb, 256, 0, TESM_LOGGED(st, mimo_coef_kernel<kF32>)>>>(mimo_x, mimo_o, H, Rm, D, coef, x0sq);
  return check_launch("mimo coef");
}

int launch_mimo_mix(const MimoMixArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "mimo mix: dtype must be 0 or 1");
  TESM_REQUIRE(a.W >= 1 && a.W <= 64 && a.H >= 1 && a.D >= 1, kErrInvalidArg, "mimo mix: bad sizes");
  TESM_REQUIRE(a.S && a.wts && a.coef && a.te && a.cc, kErrInvalidArg, "mimo mix: null pointer");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.B * a.H <= 65535 && (a.L + kMixTP - 1) / kMixTP <= 65535, kErrUnsupported, "mimo mix: grid too large");
  static_assert((kMixTP + 63) * (kMixDS / 4) <= kMixLD * 256, "state prefetch must cover the block and its halo");
  const int64_t nblk = (a.D + kMixDS - 1) / kMixDS;
  const dim3 grid(static_cast<unsigned>((nblk + kMixCB - 1) / kMixCB), static_cast<unsigned>((a.L + kMixTP - 1) / kMixTP),
                  static_cast<unsigned>(a.B * a.H));
  const size_t lds = static_cast<size_t>(((kMixTP + a.W - 1) * kMixSP + a.W * kMixWP) * sizeof(float));
  // float4 state loads and 4-wide stores need every channel group 4-aligned in memory
  const bool vec = a.D % 4 == 0 && (a.H * a.D) % 4 == 0 && reinterpret_cast<uintptr_t>(a.S) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(a.te) % (a.dt == kBF16 ? 8 : 16) == 0 &&
                   reinterpret_cast<uintptr_t>(a.cc) % (a.dt == kBF16 ? 8 : 16) == 0;
  if (a.dt == kBF16) {
    if (vec && a.W == 64) mimo_mix_kernel<kBF16, true, 64><<<grid, 256, lds, TESM_LOGGED(st, mimo_mix_kernel<kBF16, true, 64>)>>>(a);
    else if (vec) mimo_mix_kernel<kBF16, true, 0><<<grid, 256, lds, TESM_LOGGED(st, mimo_mix_kernel<kBF16, true, 0>)>>>(a);
    else mimo_mix_kernel<kBF16, false, 0><<<grid, 256, lds, TESM_LOGGED(st, mimo_mix_kernel<kBF16, false, 0>)>>>(a);
  } else {
    if (vec && a.W == 64) mimo_mix_kernel<kF32, true, 64><<<grid, 256, lds, TESM_LOGGED(st, mimo_mix_kernel<kF32, true, 64>)>>>(a);
    else if (vec) mimo_mix_kernel<kF32, true, 0><<<grid, 256, lds, TESM_LOGGED(st, mimo_mix_kernel<kF32, true, 0>)>>>(a);
    else mimo_mix_kernel<kF32, false, 0><<<grid, 256, lds, TESM_LOGGED(st, mimo_mix_kernel<kF32, false, 0>)>>>(a);
  }
  return check_launch("mimo mix");
}

int launch_mimo_final(const float* S, const float* x0sq, int64_t B, int64_t L, int64_t C, double* h_final,
                      float* last, hipStream_t st) {
  if (B == 0 || L == 0 || (!h_final && !last)) return kOk;
  TESM_REQUIRE(S && x0sq, kErrInvalidArg, "mimo final: null pointer");
  const unsigned nb = static_cast<unsigned>((B * C + 255) / 256);
  mimo_final_kernel<<<nb, 256, 0, TESM_LOGGED(st, mimo_final_kernel)>>>(S, x0sq, B, L, C, h_final, last);
  return check_launch("mimo final");
}

}  // namespace tesm
