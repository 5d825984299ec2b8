// Local-window ternary "entanglement" for gfx950.
//
// Reference (torch branch): tesm_ssm/modules/tesm.py:921-952 (SISO, `_compute_local_entanglement`),
// tesm.py:672-714 (hard ternary decision in eval), tesm.py:783-793 (RoPE), and
// tesm_ssm/modules/tesm_mimo.py:525-588 (MIMO, with its early-window truncation).
//
// For position t and window slot w (key j):
//   score = rnd(rnd(rnd(q_t . k_j) / sqrt(R)) + bias[w])       (q, k after RoPE; q + cross bias)
//   tern  = +1 if score > thr, -1 if score < -thr, else 0     (0 for keys outside the window)
//   wt    = rnd(tern / max(sum |tern|, 1))
//   avg   = rnd(sum_w wt_w * S_j)
//   E = rnd(S_t + rnd(scale * rnd(avg - S_t))),  C = rnd(E - S_t),  tanh(E)   (tesm.py:1231-1232, 1256)
// rnd() rounds to the layer dtype where the reference's torch op does.
//
// Two kernels:
//   * ent_scores_kernel: one lane per (position, window slot), a lane group per position; RoPE is
//     applied on the fly from a (L, R/2) cos/sin table; writes normalised weights (B, L, H, W).
//   * ent_mix_kernel: a workgroup per (row, 64 positions, 64 channels) stages the state halo
//     (64 + W - 1 rows) in LDS and forms the window sums, the mix and tanh in one pass.
#include "entangle.h"
#include "tesm_hip_internal.h"

namespace tesm {

namespace {

template <int DT>
__global__ __launch_bounds__(256) void rope_table_kernel(float2* __restrict__ tab, int64_t L, int64_t R,
                                                         int64_t pos_offset, double base) {
  const int64_t half = R / 2;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= L * half) return;
  const int64_t t = idx / half, i = idx - t * half;
  // inv_freq = 1 / base ** (2 * i / R) in float32 (tesm.py:787-788)
  const float e = (2.0f * static_cast<float>(i)) / static_cast<float>(R);
  const float p = static_cast<float>(pow(base, static_cast<double>(e)));
  const float inv = 1.0f / p;
  const float th = static_cast<float>(pos_offset + t) * inv;
  const double thd = static_cast<double>(th);
  tab[idx] = make_float2(rnd<DT>(static_cast<float>(cos(thd))), rnd<DT>(static_cast<float>(sin(thd))));
}

// One RoPE'd pair (x[i], x[i + R/2]) rotated by (c, s), rounded like the reference.
template <int DT>
__device__ __forceinline__ void rope_pair(float xa, float xb, float2 cs, float& o1, float& o2) {
  o1 = rnd<DT>(rnd<DT>(xa * cs.x) - rnd<DT>(xb * cs.y));
  o2 = rnd<DT>(rnd<DT>(xa * cs.y) + rnd<DT>(xb * cs.x));
}

template <int DT, int MIMO, int WP>
__global__ __launch_bounds__(256) void ent_scores_kernel(EntArgs a, int64_t weff, float inv_unused) {
  const int lane = threadIdx.x & 63;
  const int w = lane & (WP - 1);
  const int64_t gi = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) / WP;  // (b, t, h) group
  const int64_t ngroups = a.B * a.L * a.H;
  const bool in_range = gi < ngroups;
  const int64_t h = in_range ? gi % a.H : 0;
  const int64_t bt = in_range ? gi / a.H : 0;
  const int64_t t = bt % a.L, b = bt / a.L;

  int64_t j;
  bool valid;
  int bias_w;
  if constexpr (MIMO) {
    j = t - a.W + 1 + w;
    valid = in_range && w < weff && w < t + 1 && j >= 0;
    bias_w = w;
  } else {
    j = t - (weff - 1) + w;
    valid = in_range && w < weff && j >= 0;
    bias_w = static_cast<int>(a.W - weff) + w;
  }
  float tern = 0.0f;
  if (valid) {
    const int64_t half = a.R / 2;
    const int64_t qo = bt * a.ld_q + h * a.R;
    const int64_t ko = (b * a.L + j) * a.ld_k + h * a.R;
    const int64_t ao = bt * a.ld_qadd + h * a.R;
    const float2* ct = a.rope + t * half;
    const float2* cj = a.rope + j * half;
    float dot = 0.0f;
    for (int64_t i = 0; i < half; ++i) {
      float q1, q2, k1, k2;
      rope_pair<DT>(ld<DT>(a.q, qo + i), ld<DT>(a.q, qo + half + i), ct[i], q1, q2);
      if (a.q_add) {
        q1 = rnd<DT>(q1 + ld<DT>(a.q_add, ao + i));
        q2 = rnd<DT>(q2 + ld<DT>(a.q_add, ao + half + i));
      }
      rope_pair<DT>(ld<DT>(a.k, ko + i), ld<DT>(a.k, ko + half + i), cj[i], k1, k2);
      if constexpr (MIMO) {
        dot += rnd<DT>(q1 * k1);
        dot += rnd<DT>(q2 * k2);
      } else {
        dot += q1 * k1;
        dot += q2 * k2;
      }
    }
    const float sq = static_cast<float>(sqrt(static_cast<double>(a.R)));
    float s = rnd<DT>(rnd<DT>(dot) / sq);
    s = rnd<DT>(s + a.bias[h * a.W + bias_w]);
    tern = s > a.thr ? 1.0f : (s < -a.thr ? -1.0f : 0.0f);
  }
  float n = fabsf(tern);
#pragma unroll
  for (int m = WP / 2; m > 0; m >>= 1) n += __shfl_xor(n, m, 64);
  n = fmaxf(n, 1.0f);
  if (in_range && w < weff) {
    a.wts[gi * weff + w] = rnd<DT>(tern / n);
    if (a.tern) a.tern[gi * weff + w] = static_cast<int8_t>(tern);
  }
}

constexpr int kMixTP = 64;  // positions per workgroup
constexpr int kMixDS = 64;  // channels per workgroup

template <int DT>
__global__ __launch_bounds__(256) void ent_mix_kernel(EntArgs a, int64_t weff) {
  extern __shared__ float lds[];
  const int64_t rows = kMixTP + weff - 1;
  float* srow = lds;                    // [rows][kMixDS]
  float* wt = lds + rows * kMixDS;      // [kMixTP][weff]
  const int64_t bh = blockIdx.z;        // b * H + h
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t t0 = static_cast<int64_t>(blockIdx.y) * kMixTP;
  const int64_t d0 = static_cast<int64_t>(blockIdx.x) * kMixDS;
  const int c = threadIdx.x & 63;
  const int pq = threadIdx.x >> 6;
  const int64_t d = d0 + c;
  const bool dok = d < a.D;

  for (int64_t r = pq; r < rows; r += 4) {
    const int64_t t = t0 - (weff - 1) + r;
    float v = 0.0f;
    if (dok && t >= 0 && t < a.L) v = ld<DT>(a.S, (b * a.L + t) * a.ld_s + h * a.D + d);
    srow[r * kMixDS + c] = v;
  }
  for (int64_t i = threadIdx.x; i < kMixTP * weff; i += 256) {
    const int64_t p = i / weff, w = i - p * weff;
    const int64_t t = t0 + p;
    wt[i] = t < a.L ? a.wts[((b * a.L + t) * a.H + h) * weff + w] : 0.0f;
  }
  __syncthreads();
  if (!dok) return;
  for (int p = pq; p < kMixTP; p += 4) {
    const int64_t t = t0 + p;
    if (t >= a.L) break;
    float acc = 0.0f;
    for (int64_t w = 0; w < weff; ++w) acc += wt[p * weff + w] * srow[(p + w) * kMixDS + c];
    const float avg = rnd<DT>(acc);
    const float s = srow[(p + weff - 1) * kMixDS + c];
    const float e = rnd<DT>(s + rnd<DT>(a.ent_scale * rnd<DT>(avg - s)));
    const int64_t o = (b * a.L + t) * a.ld_out + h * a.D + d;
    if (a.avg) st<DT>(a.avg, o, avg);
    if (a.e_out) st<DT>(a.e_out, o, e);
    if (a.c_out) st<DT>(a.c_out, o, e - s);
    if (a.e_tanh) st<DT>(a.e_tanh, o, tanhf(e));
  }
}

template <int DT, int MIMO>
int run_scores(const EntArgs& a, int64_t weff, hipStream_t st) {
  const int64_t groups = a.B * a.L * a.H;
  auto blocks = [&](int wp) { return static_cast<unsigned>((groups * wp + 255) / 256); };
  if (weff <= 8) ent_scores_kernel<DT, MIMO, 8><<<blocks(8), 256, 0, st>>>(a, weff, 0.f);
  else if (weff <= 16) ent_scores_kernel<DT, MIMO, 16><<<blocks(16), 256, 0, st>>>(a, weff, 0.f);
  else if (weff <= 32) ent_scores_kernel<DT, MIMO, 32><<<blocks(32), 256, 0, st>>>(a, weff, 0.f);
  else ent_scores_kernel<DT, MIMO, 64><<<blocks(64), 256, 0, st>>>(a, weff, 0.f);
  return check_launch("entanglement scores");
}

template <int DT>
int run_mix(const EntArgs& a, int64_t weff, hipStream_t st) {
  dim3 grid(static_cast<unsigned>((a.D + kMixDS - 1) / kMixDS), static_cast<unsigned>((a.L + kMixTP - 1) / kMixTP),
            static_cast<unsigned>(a.B * a.H));
  const size_t lds = static_cast<size_t>((kMixTP + weff - 1) * kMixDS + kMixTP * weff) * sizeof(float);
  ent_mix_kernel<DT><<<grid, 256, lds, st>>>(a, weff);
  return check_launch("entanglement mix");
}

}  // namespace

int launch_rope_table(float2* tab, int64_t L, int64_t R, int64_t pos_offset, double base, int dt, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "rope_table: dtype must be 0 or 1");
  TESM_REQUIRE(L >= 0 && R >= 2 && R % 2 == 0 && pos_offset >= 0, kErrInvalidArg,
               "rope_table: need L >= 0, even R >= 2, pos_offset >= 0");
  if (L == 0) return kOk;
  TESM_REQUIRE(tab != nullptr, kErrInvalidArg, "rope_table: null pointer");
  const unsigned nb = static_cast<unsigned>((L * (R / 2) + 255) / 256);
  if (dt == kBF16)
    rope_table_kernel<kBF16><<<nb, 256, 0, st>>>(tab, L, R, pos_offset, base);
  else
    rope_table_kernel<kF32><<<nb, 256, 0, st>>>(tab, L, R, pos_offset, base);
  return check_launch("rope_table");
}

static int64_t eff_window(const EntArgs& a) { return a.mimo ? a.W : std::min(a.W, a.L); }

int64_t ent_ws_bytes(int64_t B, int64_t L, int64_t H, int64_t W) {
  return round_up(std::max<int64_t>(1, B * L * H * W) * static_cast<int64_t>(sizeof(float)), 256);
}

int launch_local_ent(const EntArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "local_ent: dtype must be 0 or 1");
  TESM_REQUIRE(a.B >= 0 && a.L >= 0 && a.H >= 1 && a.D >= 1, kErrInvalidArg, "local_ent: bad sizes");
  TESM_REQUIRE(a.R >= 2 && a.R % 2 == 0, kErrInvalidArg, "local_ent: ent_rank must be even (RoPE halves)");
  TESM_REQUIRE(a.W >= 1 && a.W <= 64, kErrUnsupported, "local_ent: window must be in [1, 64]");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.q && a.k && a.rope && a.bias && a.S && a.wts, kErrInvalidArg, "local_ent: null pointer");
  TESM_REQUIRE(a.ld_q >= a.H * a.R && a.ld_k >= a.H * a.R && a.ld_s >= a.H * a.D, kErrInvalidArg, "local_ent: bad ld");
  TESM_REQUIRE(!a.q_add || a.ld_qadd >= a.H * a.R, kErrInvalidArg, "local_ent: bad ld_qadd");
  TESM_REQUIRE(!(a.avg || a.e_tanh || a.c_out || a.e_out) || a.ld_out >= a.H * a.D, kErrInvalidArg,
               "local_ent: bad ld_out");
  TESM_REQUIRE(a.B * a.H <= 65535 && (a.L + kMixTP - 1) / kMixTP <= 65535, kErrUnsupported, "local_ent: grid too large");
  const int64_t weff = eff_window(a);
  int rc;
  if (a.dt == kBF16)
    rc = a.mimo ? run_scores<kBF16, 1>(a, weff, st) : run_scores<kBF16, 0>(a, weff, st);
  else
    rc = a.mimo ? run_scores<kF32, 1>(a, weff, st) : run_scores<kF32, 0>(a, weff, st);
  if (rc) return rc;
  if (!(a.avg || a.e_tanh || a.c_out || a.e_out)) return kOk;
  return a.dt == kBF16 ? run_mix<kBF16>(a, weff, st) : run_mix<kF32>(a, weff, st);
}

}  // namespace tesm
