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
  extern __shared__ float lds_mix[];
  const int64_t rows = kMixTP + weff - 1;
  float* srow = lds_mix;                // [rows][kMixDS]
  float* wt = lds_mix + rows * kMixDS;  // [kMixTP][weff]
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

// ---------------------------------------------------------------------------
// Fused SISO kernel: a workgroup per (batch row, kFusedTP positions) with all D channels, so the
// per-token quantization of tanh(E) and C happens in place.  The arithmetic of each value is the
// same sequence of float operations as in ent_scores_kernel + ent_mix_kernel.
// ---------------------------------------------------------------------------
constexpr int kFusedTP = 16;
constexpr int kFusedMaxCPD = 2;  // channels per thread: D <= 512

struct FusedLds {
  int64_t kr, qr, wt, wn, sx, red, total;  // byte offsets
  int64_t krs;                             // row stride of kr / qr in floats (R + 1: no bank conflicts)
};

__host__ __device__ inline FusedLds fused_lds(int64_t R, int64_t D, int64_t weff, int64_t ldq, int esz) {
  FusedLds f;
  const int64_t rows = kFusedTP + weff - 1;
  f.krs = R + 1;
  f.kr = 0;
  f.qr = f.kr + rows * f.krs * 4;
  const int64_t scores_end = f.qr + kFusedTP * f.krs * 4;
  const int64_t codes_end = 2 * kFusedTP * ldq;  // code staging reuses the kr/qr region
  int64_t off = ((scores_end > codes_end ? scores_end : codes_end) + 15) / 16 * 16;
  f.wt = off;
  off += kFusedTP * weff * 4;
  f.wn = off;
  off += kFusedTP * weff * 4;
  f.red = off;
  off += 2 * 2 * kFusedTP * 4 * 4;  // [amax|sum][te|c][TP][4 waves]
  off = (off + 15) / 16 * 16;
  f.sx = off;
  off += rows * D * esz;
  f.total = (off + 15) / 16 * 16;
  return f;
}

template <int DT>
__global__ __launch_bounds__(256) void ent_fused_kernel(EntArgs a, int64_t weff, FusedLds f) {
  using T = typename Elem<DT>::T;
  extern __shared__ __attribute__((aligned(16))) char lds_fused[];
  char* lds = lds_fused;
  float* kr = reinterpret_cast<float*>(lds + f.kr);
  float* qr = reinterpret_cast<float*>(lds + f.qr);
  float* wt = reinterpret_cast<float*>(lds + f.wt);
  float* wn = reinterpret_cast<float*>(lds + f.wn);
  float* red = reinterpret_cast<float*>(lds + f.red);
  T* sx = reinterpret_cast<T*>(lds + f.sx);
  int8_t* codes = reinterpret_cast<int8_t*>(lds);  // after the scores: [2][TP][ldq]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kFusedTP;
  const int64_t half = a.R / 2, R = a.R, D = a.D;
  const int64_t rows = kFusedTP + weff - 1;
  const int64_t tk0 = t0 - (weff - 1);  // position of key row 0

  // 1. RoPE'd keys and queries (tesm.py:783-793, 1209-1218)
  for (int64_t i = tid; i < rows * half; i += 256) {
    const int64_t r = i / half, c = i - r * half;
    const int64_t t = tk0 + r;
    float o1 = 0.0f, o2 = 0.0f;
    if (t >= 0 && t < a.L) {
      const int64_t ko = (b * a.L + t) * a.ld_k;
      rope_pair<DT>(ld<DT>(a.k, ko + c), ld<DT>(a.k, ko + half + c), a.rope[t * half + c], o1, o2);
    }
    kr[r * f.krs + c] = o1;
    kr[r * f.krs + half + c] = o2;
  }
  for (int64_t i = tid; i < kFusedTP * half; i += 256) {
    const int64_t p = i / half, c = i - p * half;
    const int64_t t = t0 + p;
    float o1 = 0.0f, o2 = 0.0f;
    if (t < a.L) {
      const int64_t qo = (b * a.L + t) * a.ld_q;
      rope_pair<DT>(ld<DT>(a.q, qo + c), ld<DT>(a.q, qo + half + c), a.rope[t * half + c], o1, o2);
      if (a.q_add) {
        const int64_t ao = (b * a.L + t) * a.ld_qadd;
        o1 = rnd<DT>(o1 + ld<DT>(a.q_add, ao + c));
        o2 = rnd<DT>(o2 + ld<DT>(a.q_add, ao + half + c));
      }
    }
    qr[p * f.krs + c] = o1;
    qr[p * f.krs + half + c] = o2;
  }
  // 2. state halo rows, raw dtype
  const T* S = static_cast<const T*>(a.S);
  for (int64_t i = tid; i < rows * D; i += 256) {
    const int64_t r = i / D, c = i - r * D;
    const int64_t t = tk0 + r;
    sx[i] = (t >= 0 && t < a.L) ? S[(b * a.L + t) * a.ld_s + c] : T(0);
  }
  __syncthreads();

  // 3. window scores and ternary decisions (same float sequence as ent_scores_kernel)
  const float sq = static_cast<float>(sqrt(static_cast<double>(R)));
  for (int64_t i = tid; i < kFusedTP * weff; i += 256) {
    const int64_t p = i / weff, w = i - p * weff;
    const int64_t t = t0 + p, j = t - (weff - 1) + w;
    float tern = 0.0f;
    if (t < a.L && j >= 0) {
      const float* qp = qr + p * f.krs;
      const float* kp = kr + (p + w) * f.krs;
      float dot = 0.0f;
      for (int64_t c = 0; c < half; ++c) {
        dot += qp[c] * kp[c];
        dot += qp[half + c] * kp[half + c];
      }
      float s = rnd<DT>(rnd<DT>(dot) / sq);
      s = rnd<DT>(s + a.bias[a.W - weff + w]);
      tern = s > a.thr ? 1.0f : (s < -a.thr ? -1.0f : 0.0f);
    }
    wt[i] = tern;
    if (a.tern && t < a.L) a.tern[(b * a.L + t) * weff + w] = static_cast<int8_t>(tern);
  }
  __syncthreads();
  for (int64_t i = tid; i < kFusedTP * weff; i += 256) {
    const int64_t p = i / weff;
    float n = 0.0f;
    for (int64_t w = 0; w < weff; ++w) n += fabsf(wt[p * weff + w]);
    n = fmaxf(n, 1.0f);
    wn[i] = rnd<DT>(wt[i] / n);
  }
  // zero the code staging area (it overlays kr/qr, free after the scores)
  for (int64_t i = tid; i < 2 * kFusedTP * a.ldq / 16; i += 256)
    reinterpret_cast<uint4*>(codes)[i] = make_uint4(0, 0, 0, 0);
  __syncthreads();

  // 4. window average, mix, tanh (ent_mix_kernel arithmetic), held in registers
  float te[kFusedTP][kFusedMaxCPD], cc[kFusedTP][kFusedMaxCPD];
  float mx_te[kFusedTP], mx_c[kFusedTP];
#pragma unroll
  for (int p = 0; p < kFusedTP; ++p) {
    mx_te[p] = 0.0f;
    mx_c[p] = 0.0f;
#pragma unroll
    for (int jj = 0; jj < kFusedMaxCPD; ++jj) {
      te[p][jj] = 0.0f;
      cc[p][jj] = 0.0f;
      const int64_t c = tid + 256 * jj;
      const int64_t t = t0 + p;
      if (c >= D || t >= a.L) continue;
      float acc = 0.0f;
      for (int64_t w = 0; w < weff; ++w) acc += wn[p * weff + w] * ld<DT>(sx, (p + w) * D + c);
      const float avg = rnd<DT>(acc);
      const float s = ld<DT>(sx, (p + weff - 1) * D + c);
      const float e = rnd<DT>(s + rnd<DT>(a.ent_scale * rnd<DT>(avg - s)));
      const float cv = rnd<DT>(e - s);
      const float tv = rnd<DT>(tanhf(e));
      const int64_t o = (b * a.L + t) * a.ld_out + c;
      if (a.avg) st<DT>(a.avg, o, avg);
      if (a.e_out) st<DT>(a.e_out, o, e);
      if (a.c_out) st<DT>(a.c_out, o, cv);
      if (a.e_tanh) st<DT>(a.e_tanh, o, tv);
      te[p][jj] = tv;
      cc[p][jj] = cv;
      mx_te[p] = fmaxf(mx_te[p], fabsf(tv));
      mx_c[p] = fmaxf(mx_c[p], fabsf(cv));
    }
  }
  // 5. per-token scales (tesm.py:206-209) over the D channels of the workgroup
#pragma unroll
  for (int p = 0; p < kFusedTP; ++p) {
    const float m1 = wave_max(mx_te[p]), m2 = wave_max(mx_c[p]);
    if (lane == 0) {
      red[(0 * kFusedTP + p) * 4 + wave] = m1;
      red[(1 * kFusedTP + p) * 4 + wave] = m2;
    }
  }
  __syncthreads();
  float sc_te[kFusedTP], sc_c[kFusedTP];
#pragma unroll
  for (int p = 0; p < kFusedTP; ++p) {
    const float* r0 = red + (0 * kFusedTP + p) * 4;
    const float* r1 = red + (1 * kFusedTP + p) * 4;
    sc_te[p] = act_scale<DT>(fmaxf(fmaxf(r0[0], r0[1]), fmaxf(r0[2], r0[3])), a.eps);
    sc_c[p] = act_scale<DT>(fmaxf(fmaxf(r1[0], r1[1]), fmaxf(r1[2], r1[3])), a.eps);
  }
  // 6. codes into the staging rows, row sums of the codes
  int32_t* redi = reinterpret_cast<int32_t*>(red + 2 * kFusedTP * 4);
  __syncthreads();  // everyone has read red[] before it is reused for the sums
#pragma unroll
  for (int p = 0; p < kFusedTP; ++p) {
    int s1 = 0, s2 = 0;
#pragma unroll
    for (int jj = 0; jj < kFusedMaxCPD; ++jj) {
      const int64_t c = tid + 256 * jj;
      if (c >= D || t0 + p >= a.L) continue;
      const int q1 = act_code<DT>(te[p][jj], sc_te[p]);
      const int q2 = act_code<DT>(cc[p][jj], sc_c[p]);
      const int64_t pos = (c & ~15) + layout1_pos(static_cast<int>(c & 15));
      codes[(0 * kFusedTP + p) * a.ldq + pos] = static_cast<int8_t>(q1);
      codes[(1 * kFusedTP + p) * a.ldq + pos] = static_cast<int8_t>(q2);
      s1 += q1;
      s2 += q2;
    }
    s1 = wave_sum_i(s1);
    s2 = wave_sum_i(s2);
    if (lane == 0) {
      redi[(0 * kFusedTP + p) * 4 + wave] = s1;
      redi[(1 * kFusedTP + p) * 4 + wave] = s2;
    }
  }
  __syncthreads();
  if (tid < 2 * kFusedTP) {
    const int which = tid / kFusedTP, p = tid % kFusedTP;
    const int64_t t = t0 + p;
    if (t < a.L) {
      const int32_t* r = redi + (which * kFusedTP + p) * 4;
      const int64_t row = b * a.L + t;
      if (which == 0) {
        a.s_te[row] = sc_te[p];
        a.rs_te[row] = (r[0] + r[1]) + (r[2] + r[3]);
      } else {
        a.s_c[row] = sc_c[p];
        a.rs_c[row] = (r[0] + r[1]) + (r[2] + r[3]);
      }
    }
  }
  const int64_t chunks = a.ldq / 16;
  for (int64_t i = tid; i < 2 * kFusedTP * chunks; i += 256) {
    const int64_t rr = i / chunks, ck = i - rr * chunks;
    const int which = static_cast<int>(rr / kFusedTP), p = static_cast<int>(rr % kFusedTP);
    const int64_t t = t0 + p;
    if (t >= a.L) continue;
    int8_t* dst = (which == 0 ? a.q_te : a.q_c) + (b * a.L + t) * a.ldq + 16 * ck;
    *reinterpret_cast<uint4*>(dst) = reinterpret_cast<const uint4*>(codes + rr * a.ldq)[ck];
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

bool ent_fused_ok(const EntArgs& a) {
  if (a.mimo || a.H != 1 || a.D > 256 * kFusedMaxCPD) return false;
  const int64_t weff = eff_window(a);
  const int64_t ldq = a.ldq > 0 ? a.ldq : kpad(a.D);
  return fused_lds(a.R, a.D, weff, ldq, a.dt == kBF16 ? 2 : 4).total <= 64 * 1024;
}

int64_t ent_ws_bytes(int64_t B, int64_t L, int64_t H, int64_t W) {
  return round_up(std::max<int64_t>(1, B * L * H * W) * static_cast<int64_t>(sizeof(float)), 256);
}

int launch_local_ent(const EntArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "local_ent: dtype must be 0 or 1");
  TESM_REQUIRE(a.B >= 0 && a.L >= 0 && a.H >= 1 && a.D >= 1, kErrInvalidArg, "local_ent: bad sizes");
  TESM_REQUIRE(a.R >= 2 && a.R % 2 == 0, kErrInvalidArg, "local_ent: ent_rank must be even (RoPE halves)");
  TESM_REQUIRE(a.W >= 1 && a.W <= 64, kErrUnsupported, "local_ent: window must be in [1, 64]");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.q && a.k && a.rope && a.bias && a.S, kErrInvalidArg, "local_ent: null pointer");
  TESM_REQUIRE(a.q_te || a.wts, kErrWorkspace, "local_ent: missing window-weight workspace");
  TESM_REQUIRE(a.ld_q >= a.H * a.R && a.ld_k >= a.H * a.R && a.ld_s >= a.H * a.D, kErrInvalidArg, "local_ent: bad ld");
  TESM_REQUIRE(!a.q_add || a.ld_qadd >= a.H * a.R, kErrInvalidArg, "local_ent: bad ld_qadd");
  TESM_REQUIRE(!(a.avg || a.e_tanh || a.c_out || a.e_out) || a.ld_out >= a.H * a.D, kErrInvalidArg,
               "local_ent: bad ld_out");
  TESM_REQUIRE(a.B * a.H <= 65535 && (a.L + kMixTP - 1) / kMixTP <= 65535, kErrUnsupported, "local_ent: grid too large");
  const int64_t weff = eff_window(a);
  if (a.q_te) {
    TESM_REQUIRE(ent_fused_ok(a), kErrUnsupported,
                 "local_ent: fused quantization needs SISO, D <= 512 and a small enough window/rank");
    TESM_REQUIRE(a.q_c && a.s_te && a.s_c && a.rs_te && a.rs_c && a.ldq >= a.D && a.ldq % 16 == 0 &&
                     aligned(a.q_te, 16) && aligned(a.q_c, 16),
                 kErrInvalidArg, "local_ent: bad quantized outputs");
    const FusedLds f = fused_lds(a.R, a.D, weff, a.ldq, a.dt == kBF16 ? 2 : 4);
    dim3 grid(static_cast<unsigned>((a.L + kFusedTP - 1) / kFusedTP), static_cast<unsigned>(a.B));
    if (a.dt == kBF16)
      ent_fused_kernel<kBF16><<<grid, 256, f.total, st>>>(a, weff, f);
    else
      ent_fused_kernel<kF32><<<grid, 256, f.total, st>>>(a, weff, f);
    return check_launch("entanglement fused");
  }
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
