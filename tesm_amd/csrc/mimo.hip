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

constexpr int kMimoTP = 64;  // positions per workgroup
constexpr int kMimoDS = 64;  // channels per workgroup

// Window mix for one (batch row, head) pair, kMimoTP positions x kMimoDS channels: key position of
// window slot w is t - W + 1 + w (tesm_mimo.py:536-586); slots the reference drops carry weight 0.
template <int DT>
__global__ __launch_bounds__(256) void mimo_mix_kernel(MimoMixArgs a) {
  extern __shared__ float lds_mimo[];
  const int64_t W = a.W;
  const int64_t rows = kMimoTP + W - 1;
  float* srow = lds_mimo;                 // [rows][kMimoDS]
  float* wt = lds_mimo + rows * kMimoDS;  // [kMimoTP][W]
  const int64_t bh = blockIdx.z;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kMimoTP;
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kMimoDS;
  const int c = threadIdx.x & 63, pq = threadIdx.x >> 6;
  const int64_t d = d0 + c;
  const bool dok = d < a.D;
  const int64_t C = a.H * a.D;
  for (int64_t r = pq; r < rows; r += 4) {
    const int64_t t = t0 - (W - 1) + r;
    srow[r * kMimoDS + c] = (dok && t >= 0 && t < a.L) ? a.S[(b * a.L + t) * C + h * a.D + d] : 0.0f;
  }
  for (int64_t i = threadIdx.x; i < kMimoTP * W; i += 256) {
    const int64_t p = i / W, w = i - p * W;
    const int64_t t = t0 + p;
    wt[i] = t < a.L ? a.wts[((b * a.L + t) * a.H + h) * W + w] : 0.0f;
  }
  __syncthreads();
  if (!dok) return;
  const float cf = a.coef[h * a.D + d];
  for (int p = pq; p < kMimoTP; p += 4) {
    const int64_t t = t0 + p;
    if (t >= a.L) break;
    float acc = 0.0f;
    for (int64_t w = 0; w < W; ++w) acc += wt[p * W + w] * srow[(p + w) * kMimoDS + c];
    const float s = srow[(p + W - 1) * kMimoDS + c];
    const float e = s + a.ent_scale * (acc - s);
    const float ch = e - s;
    const int64_t o = (b * a.L + t) * C + h * a.D + d;
    st<DT>(a.te, o, tanhf_(e * cf));
    st<DT>(a.cc, o, ch * cf);
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
  const int64_t V = a.S - a.W + 1, half = a.R / 2;
  const int64_t n = V * a.H * a.W;
  int32_t pos = 0, neg = 0;
  for (int64_t e = threadIdx.x; e < n; e += 256) {
    const int64_t v = e / (a.H * a.W), h = (e / a.W) % a.H, w = e % a.W;
    const int64_t tq = a.W - 1 + v, tk = v + w;
    const int64_t qo = (b * a.L + tq) * a.ld_q + h * a.R, ko = (b * a.L + tk) * a.ld_k + h * a.R;
    float acc = 0.0f;
    for (int part = 0; part < 2; ++part) {
      for (int64_t i = 0; i < half; ++i) {
        float q1, q2, k1, k2;
        rope_pair<DT>(ld<DT>(a.q, qo + i), ld<DT>(a.q, qo + i + half), a.rope[tq * half + i], q1, q2);
        rope_pair<DT>(ld<DT>(a.k, ko + i), ld<DT>(a.k, ko + i + half), a.rope[tk * half + i], k1, k2);
        acc += part == 0 ? rnd<DT>(q1 * k1) : rnd<DT>(q2 * k2);
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
  TESM_REQUIRE(a.W >= 1 && a.S >= a.W && a.S <= a.L && a.R >= 2 && a.R % 2 == 0 && a.H >= 1, kErrInvalidArg,
               "mimo stats: need 1 <= W <= S <= L and an even R");
  TESM_REQUIRE((a.S - a.W + 1) * a.H * a.W <= 0x7fffffff, kErrUnsupported, "mimo stats: too many scores");
  if (a.dt == kBF16)
    mimo_stats_kernel<kBF16><<<static_cast<unsigned>(a.B), 256, 0, st>>>(a);
  else
    mimo_stats_kernel<kF32><<<static_cast<unsigned>(a.B), 256, 0, st>>>(a);
  return check_launch("mimo stats");
}

int launch_mimo_coef(const void* mimo_x, const void* mimo_o, int dt, int64_t H, int64_t Rm, int64_t D, float* coef,
                     float* x0sq, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "mimo coef: dtype must be 0 or 1");
  TESM_REQUIRE(H >= 1 && Rm >= 1 && D >= 1, kErrInvalidArg, "mimo coef: bad sizes");
  TESM_REQUIRE(mimo_x && mimo_o && coef && x0sq, kErrInvalidArg, "mimo coef: null pointer");
  const unsigned nb = static_cast<unsigned>((H * D + 255) / 256);
  if (dt == kBF16)
    mimo_coef_kernel<kBF16><<<nb, 256, 0, st>>>(mimo_x, mimo_o, H, Rm, D, coef, x0sq);
  else
    mimo_coef_kernel<kF32><<<nb, 256, 0, st>>>(mimo_x, mimo_o, H, Rm, D, coef, x0sq);
  return check_launch("mimo coef");
}

int launch_mimo_mix(const MimoMixArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "mimo mix: dtype must be 0 or 1");
  TESM_REQUIRE(a.W >= 1 && a.W <= 64 && a.H >= 1 && a.D >= 1, kErrInvalidArg, "mimo mix: bad sizes");
  TESM_REQUIRE(a.S && a.wts && a.coef && a.te && a.cc, kErrInvalidArg, "mimo mix: null pointer");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.B * a.H <= 65535 && (a.L + kMimoTP - 1) / kMimoTP <= 65535, kErrUnsupported, "mimo mix: grid too large");
  const dim3 grid(static_cast<unsigned>((a.D + kMimoDS - 1) / kMimoDS), static_cast<unsigned>((a.L + kMimoTP - 1) / kMimoTP),
                  static_cast<unsigned>(a.B * a.H));
  const size_t lds = static_cast<size_t>(((kMimoTP + a.W - 1) * kMimoDS + kMimoTP * a.W) * sizeof(float));
  if (a.dt == kBF16)
    mimo_mix_kernel<kBF16><<<grid, 256, lds, st>>>(a);
  else
    mimo_mix_kernel<kF32><<<grid, 256, lds, st>>>(a);
  return check_launch("mimo mix");
}

int launch_mimo_final(const float* S, const float* x0sq, int64_t B, int64_t L, int64_t C, double* h_final,
                      float* last, hipStream_t st) {
  if (B == 0 || L == 0 || (!h_final && !last)) return kOk;
  TESM_REQUIRE(S && x0sq, kErrInvalidArg, "mimo final: null pointer");
  const unsigned nb = static_cast<unsigned>((B * C + 255) / 256);
  mimo_final_kernel<<<nb, 256, 0, st>>>(S, x0sq, B, L, C, h_final, last);
  return check_launch("mimo final");
}

}  // namespace tesm
