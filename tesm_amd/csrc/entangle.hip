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
#include <cstdlib>

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

// ---------------------------------------------------------------------------
// MIMO window scores, tiled (tesm_mimo.py:536-586): a workgroup per (batch row, head, kScTP
// positions).  RoPE'd q rows and the key rows the window reaches (kScTP + W - 1 of them) are
// staged in LDS 32 RoPE pairs at a time, so each q / k element is rotated once per workgroup;
// each thread accumulates a 4-position x 4-window-slot tile of dot products (products rounded to
// dt before the sum, as the reference's (q * k).sum(-1) in dt).  Same arithmetic as
// ent_scores_kernel<DT, 1, .>.
// ---------------------------------------------------------------------------
constexpr int kScTP = 64;        // positions per workgroup
constexpr int kScPairs = 32;     // RoPE pairs per LDS slice (64 values per row)
constexpr int kScPitch = 2 * kScPairs;  // row pitch (floats); 16-byte chunks XOR-swizzled per 4 rows

// LDS position of column c of staged row r: the row's 16 four-column chunks are permuted by (r / 4) % 16,
// so the 16 lanes of a pass reading rows 4 apart (the window's key rows) hit 16 different bank groups
__device__ __forceinline__ int sc_col(int r, int c) { return 4 * ((c >> 2) ^ ((r >> 2) & 15)) + (c & 3); }

template <int DT>
__global__ __launch_bounds__(256) void ent_scores_mimo_kernel(EntArgs a) {
  extern __shared__ float lds_sc[];
  const int W = static_cast<int>(a.W);
  const int krows = kScTP + W - 1;
  float* qs = lds_sc;                    // [kScTP][kScPitch]
  float* ks = qs + kScTP * kScPitch;     // [krows][kScPitch]
  float* tt = lds_sc;                    // after the dots: [kScTP][W] ternary values
  float* nrm = ks;                       // after the dots: [kScTP] norms
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.H, h = bh - b * a.H;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kScTP;
  const int64_t tk0 = t0 - (W - 1);      // position of staged key row 0
  const int half = static_cast<int>(a.R / 2);
  const int nwt = (W + 3) / 4;           // 4-slot tiles along the window
  const int tile = tid;                  // tile = pg * nwt + wg
  const int pg = tile / nwt, wg = tile - pg * nwt;
  const bool active = pg < kScTP / 4;
  const int p0 = 4 * pg, w0 = 4 * wg;
  float dot[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) dot[i][j] = 0.0f;
  float wb[4];  // window bias of the thread's slots, read up front
#pragma unroll
  for (int j = 0; j < 4; ++j) wb[j] = a.bias[h * a.W + (w0 + j < W ? w0 + j : W - 1)];

  for (int i0 = 0; i0 < half; i0 += kScPairs) {
    const int np = half - i0 < kScPairs ? half - i0 : kScPairs;
    // stage RoPE'd pairs (interleaved q1, q2 per pair) of the slice: each thread loads kSB items
    // (clamped into range, raw bits) before it rotates and stores any of them
    constexpr int kSB = 8;
    const int nitems = (kScTP + krows) * kScPairs;
    for (int base = 0; base < nitems; base += 256 * kSB) {
      uint32_t xa[kSB], xb[kSB];
      float2 cs[kSB];
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        int idx = base + tid + 256 * u;
        idx = idx < nitems ? idx : nitems - 1;
        const int r = idx / kScPairs, i = idx - r * kScPairs, ic = i < np ? i : np - 1;
        const bool isq = r < kScTP;
        int64_t tt_ = isq ? t0 + r : tk0 + (r - kScTP);
        tt_ = tt_ < 0 ? 0 : (tt_ >= a.L ? a.L - 1 : tt_);
        const void* src = isq ? a.q : a.k;
        const int64_t off = (b * a.L + tt_) * (isq ? a.ld_q : a.ld_k) + h * a.R + i0 + ic;
        xa[u] = ld_bits<DT>(src, off);
        xb[u] = ld_bits<DT>(src, off + half);
        cs[u] = a.rope[tt_ * half + i0 + ic];
      }
#pragma unroll
      for (int u = 0; u < kSB; ++u) {
        const int idx = base + tid + 256 * u;
        if (idx >= nitems) break;
        const int r = idx / kScPairs, i = idx - r * kScPairs;
        const bool isq = r < kScTP;
        const int rr = isq ? r : r - kScTP;
        const int64_t tt_ = isq ? t0 + rr : tk0 + rr;
        const bool ok = i < np && tt_ >= 0 && tt_ < a.L;
        float o1 = 0.0f, o2 = 0.0f;
        if (ok) rope_pair<DT>(from_bits<DT>(xa[u]), from_bits<DT>(xb[u]), cs[u], o1, o2);
        *reinterpret_cast<float2*>((isq ? qs : ks) + rr * kScPitch + sc_col(rr, 2 * i)) = make_float2(o1, o2);
      }
    }
    __syncthreads();
    if (active) {
      // four columns per step (16-byte reads); each product added in increasing column order as before
      const int nc4 = (2 * np) >> 2;
      for (int c4 = 0; c4 < nc4; ++c4) {
        float4 qv[4], kv[7];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = p0 + i;
          qv[i] = *reinterpret_cast<const float4*>(qs + r * kScPitch + sc_col(r, 4 * c4));
        }
#pragma unroll
        for (int i = 0; i < 7; ++i) {
          const int r = p0 + w0 + i, rc = r < krows ? r : krows - 1;
          const float4 v = *reinterpret_cast<const float4*>(ks + rc * kScPitch + sc_col(rc, 4 * c4));
          kv[i] = r < krows ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const float* qf = reinterpret_cast<const float*>(&qv[i]);
              const float* kf = reinterpret_cast<const float*>(&kv[i + j]);
              dot[i][j] += rnd<DT>(qf[e] * kf[e]);
            }
      }
      for (int c = 4 * nc4; c < 2 * np; ++c) {
        float qv[4], kv[7];
#pragma unroll
        for (int i = 0; i < 4; ++i) qv[i] = qs[(p0 + i) * kScPitch + sc_col(p0 + i, c)];
#pragma unroll
        for (int i = 0; i < 7; ++i) {
          const int r = p0 + w0 + i, rc = r < krows ? r : krows - 1;
          const float v = ks[rc * kScPitch + sc_col(rc, c)];
          kv[i] = r < krows ? v : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) dot[i][j] += rnd<DT>(qv[i] * kv[i + j]);
      }
    }
    __syncthreads();
  }
  // scores, strict ternary and validity (tesm_mimo.py:540-560)
  const float sq = static_cast<float>(sqrt(static_cast<double>(a.R)));
  if (active) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t t = t0 + p0 + i;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int w = w0 + j;
        if (w >= W) continue;
        const int64_t jk = t - W + 1 + w;
        const bool valid = t < a.L && w < t + 1 && jk >= 0;
        float tern = 0.0f;
        if (valid) {
          float sc = rnd<DT>(rnd<DT>(dot[i][j]) / sq);
          sc = rnd<DT>(sc + wb[j]);
          tern = sc > a.thr ? 1.0f : (sc < -a.thr ? -1.0f : 0.0f);
        }
        tt[(p0 + i) * W + w] = tern;
      }
    }
  }
  __syncthreads();
  if (tid < kScTP) {
    float n = 0.0f;
    for (int w = 0; w < W; ++w) n += fabsf(tt[tid * W + w]);
    nrm[tid] = fmaxf(n, 1.0f);
  }
  __syncthreads();
  for (int idx = tid; idx < kScTP * W; idx += 256) {
    const int p = idx / W, w = idx - p * W;
    const int64_t t = t0 + p;
    if (t >= a.L) continue;
    const int64_t o = ((b * a.L + t) * a.H + h) * W + w;
    const float tv = tt[idx];
    a.wts[o] = rnd<DT>(tv / nrm[p]);
    if (a.tern) a.tern[o] = static_cast<int8_t>(tv);
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
    if (a.e_tanh) st<DT>(a.e_tanh, o, tanhf_(e));
  }
}

// ---------------------------------------------------------------------------
// Fused SISO kernel: a workgroup per (batch row, kFusedTP positions) with all D channels, so the
// per-token quantization of tanh(E) and C happens in place.  Thread (p, g) owns position p and
// 16-channel groups g, g + 16, ...: its window weights, window sums, mix and the 16 int8 codes of
// a group (one 16-byte store) stay in registers; row maxima and code sums reduce over the 16
// lanes of a position.  Every value is the same sequence of float operations as in
// ent_scores_kernel + ent_mix_kernel.
// ---------------------------------------------------------------------------
constexpr int kFusedTP = 16;
constexpr int kFusedMaxGPT = 2;  // channel groups per thread: D <= 16 * 16 * 2 = 512

struct FusedLds {
  int64_t kr, qr, wn, sx, total;  // byte offsets
  int64_t krs;                    // row stride of kr / qr in floats
  int64_t dp;                     // row stride of sx in elements (D rounded up to 16)
};

__host__ __device__ inline FusedLds fused_lds(int64_t R, int64_t D, int64_t weff, int esz) {
  FusedLds f;
  const int64_t rows = kFusedTP + weff - 1;
  f.krs = R + 4;
  f.dp = (D + 15) / 16 * 16;
  f.kr = 0;
  f.qr = f.kr + rows * f.krs * 4;
  f.wn = f.qr + kFusedTP * f.krs * 4;
  f.sx = (f.wn + kFusedTP * weff * 4 + 15) / 16 * 16;
  f.total = (f.sx + rows * f.dp * esz + 15) / 16 * 16;
  return f;
}

// 16 channels of one staged state row as floats.
template <int DT>
__device__ __forceinline__ void lds_row16(const void* base, float (&x)[16]) {
  if constexpr (DT == kBF16) {
    const uint4 a = reinterpret_cast<const uint4*>(base)[0], b = reinterpret_cast<const uint4*>(base)[1];
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[2 * i] = __uint_as_float(w[i] << 16);
      x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 v = reinterpret_cast<const float4*>(base)[i];
      x[4 * i] = v.x;
      x[4 * i + 1] = v.y;
      x[4 * i + 2] = v.z;
      x[4 * i + 3] = v.w;
    }
  }
}

// SI: items per thread of the single-issue load path (keys and state vectors; queries SI / 2).
template <int DT, int SI>
__global__ __launch_bounds__(256) void ent_fused_kernel(EntArgs a, int64_t weff, FusedLds f) {
  using T = typename Elem<DT>::T;
  extern __shared__ __attribute__((aligned(16))) char lds_fused[];
  float* kr = reinterpret_cast<float*>(lds_fused + f.kr);
  float* qr = reinterpret_cast<float*>(lds_fused + f.qr);
  float* wn = reinterpret_cast<float*>(lds_fused + f.wn);
  T* sx = reinterpret_cast<T*>(lds_fused + f.sx);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kFusedTP;
  const int half = static_cast<int>(a.R / 2), D = static_cast<int>(a.D), W = static_cast<int>(weff);
  const int krs = static_cast<int>(f.krs), dp = static_cast<int>(f.dp);
  const int rows = kFusedTP + W - 1;
  const int64_t tk0 = t0 - (W - 1);  // position of key row 0

  // window bias of the thread's score slots w = (tid & 15) + 16 i, read before the tile's other
  // operands (used after the LDS phase, so never waited for on its own)
  float wbias[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int w = (tid & 15) + 16 * i;
    wbias[i] = a.bias[a.W - W + (w < W ? w : W - 1)];
  }

  const T* S = static_cast<const T*>(a.S);
  constexpr int kVec = 16 / sizeof(T);
  const bool vec = (D % kVec) == 0 && (a.ld_s % kVec) == 0 && (reinterpret_cast<uintptr_t>(S) % 16) == 0;
  // Single-issue path: when the tile's keys, queries and state halo fit kKPT / kQPT / kSPT items per
  // thread, every global operand is requested before any is used (one memory round trip per tile),
  // items numbered flat over the workgroup so that all lanes take part.
  constexpr int kKPT = SI, kQPT = SI / 2, kSPT = SI;
  const int nvec = dp / kVec;
  if (vec && rows * half <= 256 * kKPT && kFusedTP * half <= 256 * kQPT && rows * nvec <= 256 * kSPT) {
    float kxa[kKPT], kxb[kKPT], qxa[kQPT], qxb[kQPT], qaa[kQPT], qab[kQPT];
    float2 kcs[kKPT], qcs[kQPT];
    v4i sv[kSPT];
#pragma unroll
    for (int k = 0; k < kSPT; ++k) {
      const int i = tid + 256 * k;
      const int r = i / nvec, c = (i - r * nvec) * kVec;
      const int cc = c < D ? c : D - kVec;
      int64_t tt = tk0 + (r < rows ? r : rows - 1);
      tt = tt < 0 ? 0 : (tt >= a.L ? a.L - 1 : tt);
      sv[k] = *reinterpret_cast<const v4i*>(S + (b * a.L + tt) * a.ld_s + cc);
    }
#pragma unroll
    for (int k = 0; k < kKPT; ++k) {
      const int i = tid + 256 * k;
      const int r = i / half, c = i - r * half;
      int64_t tt = tk0 + (r < rows ? r : rows - 1);
      tt = tt < 0 ? 0 : (tt >= a.L ? a.L - 1 : tt);
      const int64_t ko = (b * a.L + tt) * a.ld_k;
      kxa[k] = ld<DT>(a.k, ko + c);
      kxb[k] = ld<DT>(a.k, ko + half + c);
      kcs[k] = a.rope[tt * half + c];
    }
#pragma unroll
    for (int k = 0; k < kQPT; ++k) {
      const int i = tid + 256 * k;
      const int pp = i / half, c = i - pp * half;
      const int64_t tt = (t0 + pp < a.L) ? t0 + pp : a.L - 1;
      const int64_t qo = (b * a.L + tt) * a.ld_q;
      qxa[k] = ld<DT>(a.q, qo + c);
      qxb[k] = ld<DT>(a.q, qo + half + c);
      qcs[k] = a.rope[tt * half + c];
      qaa[k] = qab[k] = 0.0f;
      if (a.q_add) {
        const int64_t ao = (b * a.L + tt) * a.ld_qadd;
        qaa[k] = ld<DT>(a.q_add, ao + c);
        qab[k] = ld<DT>(a.q_add, ao + half + c);
      }
    }
#pragma unroll
    for (int k = 0; k < kSPT; ++k) {
      const int i = tid + 256 * k;
      const int r = i / nvec, c = (i - r * nvec) * kVec;
      if (r >= rows) break;
      const int64_t tt = tk0 + r;
      const bool ok = tt >= 0 && tt < a.L && c < D;
      *reinterpret_cast<v4i*>(sx + static_cast<int64_t>(r) * dp + c) = ok ? sv[k] : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < kKPT; ++k) {
      const int i = tid + 256 * k;
      const int r = i / half, c = i - r * half;
      if (r >= rows) break;
      const int64_t tt = tk0 + r;
      float o1 = 0.0f, o2 = 0.0f;
      if (tt >= 0 && tt < a.L) rope_pair<DT>(kxa[k], kxb[k], kcs[k], o1, o2);
      kr[r * krs + c] = o1;
      kr[r * krs + half + c] = o2;
    }
#pragma unroll
    for (int k = 0; k < kQPT; ++k) {
      const int i = tid + 256 * k;
      const int pp = i / half, c = i - pp * half;
      if (pp >= kFusedTP) break;
      float o1 = 0.0f, o2 = 0.0f;
      if (t0 + pp < a.L) {
        rope_pair<DT>(qxa[k], qxb[k], qcs[k], o1, o2);
        if (a.q_add) {
          o1 = rnd<DT>(o1 + qaa[k]);
          o2 = rnd<DT>(o2 + qab[k]);
        }
      }
      qr[pp * krs + c] = o1;
      qr[pp * krs + half + c] = o2;
    }
  } else {
    // 1. RoPE'd keys and queries (tesm.py:783-793, 1209-1218).  Rows go over waves, RoPE pairs over
    //    lanes; each wave loads kBatch rows (clamped into [0, L)) before it writes any of them, so the
    //    loads of a batch are in flight together.
    constexpr int kBatch = 8;
    for (int c = lane; c < half; c += 64) {
      for (int r0 = wave; r0 < rows; r0 += 4 * kBatch) {
        float xa[kBatch], xb[kBatch];
        float2 cs[kBatch];
#pragma unroll
        for (int bi = 0; bi < kBatch; ++bi) {
          int64_t tt = tk0 + r0 + 4 * bi;
          tt = tt < 0 ? 0 : (tt >= a.L ? a.L - 1 : tt);
          const int64_t ko = (b * a.L + tt) * a.ld_k;
          xa[bi] = ld<DT>(a.k, ko + c);
          xb[bi] = ld<DT>(a.k, ko + half + c);
          cs[bi] = a.rope[tt * half + c];
        }
#pragma unroll
        for (int bi = 0; bi < kBatch; ++bi) {
          const int r = r0 + 4 * bi;
          if (r >= rows) break;
          const int64_t tt = tk0 + r;
          float o1 = 0.0f, o2 = 0.0f;
          if (tt >= 0 && tt < a.L) rope_pair<DT>(xa[bi], xb[bi], cs[bi], o1, o2);
          kr[r * krs + c] = o1;
          kr[r * krs + half + c] = o2;
        }
      }
      {
        float xa[4], xb[4], qa[4], qb[4];
        float2 cs[4];
#pragma unroll
        for (int bi = 0; bi < 4; ++bi) {  // kFusedTP / 4 rows per wave
          const int pp = wave + 4 * bi;
          const int64_t tt = (t0 + pp < a.L) ? t0 + pp : a.L - 1;
          const int64_t qo = (b * a.L + tt) * a.ld_q;
          xa[bi] = ld<DT>(a.q, qo + c);
          xb[bi] = ld<DT>(a.q, qo + half + c);
          cs[bi] = a.rope[tt * half + c];
          if (a.q_add) {
            const int64_t ao = (b * a.L + tt) * a.ld_qadd;
            qa[bi] = ld<DT>(a.q_add, ao + c);
            qb[bi] = ld<DT>(a.q_add, ao + half + c);
          }
        }
#pragma unroll
        for (int bi = 0; bi < 4; ++bi) {
          const int pp = wave + 4 * bi;
          float o1 = 0.0f, o2 = 0.0f;
          if (t0 + pp < a.L) {
            rope_pair<DT>(xa[bi], xb[bi], cs[bi], o1, o2);
            if (a.q_add) {
              o1 = rnd<DT>(o1 + qa[bi]);
              o2 = rnd<DT>(o2 + qb[bi]);
            }
          }
          qr[pp * krs + c] = o1;
          qr[pp * krs + half + c] = o2;
        }
      }
    }
    // 2. state halo rows in the raw dtype, channels padded with zeros to a multiple of 16
    if (vec) {
      for (int c = lane * kVec; c < dp; c += 64 * kVec) {
        const int cc = c < D ? c : D - kVec;
        for (int r0 = wave; r0 < rows; r0 += 4 * kBatch) {
          v4i v[kBatch];
#pragma unroll
          for (int bi = 0; bi < kBatch; ++bi) {
            int64_t tt = tk0 + r0 + 4 * bi;
            tt = tt < 0 ? 0 : (tt >= a.L ? a.L - 1 : tt);
            v[bi] = *reinterpret_cast<const v4i*>(S + (b * a.L + tt) * a.ld_s + cc);
          }
#pragma unroll
          for (int bi = 0; bi < kBatch; ++bi) {
            const int r = r0 + 4 * bi;
            if (r >= rows) break;
            const int64_t tt = tk0 + r;
            const bool ok = tt >= 0 && tt < a.L && c < D;
            *reinterpret_cast<v4i*>(sx + static_cast<int64_t>(r) * dp + c) = ok ? v[bi] : v4i{0, 0, 0, 0};
          }
        }
      }
    } else {
      for (int r = wave; r < rows; r += 4) {
        const int64_t tt = tk0 + r;
        const bool ok = tt >= 0 && tt < a.L;
        const T* src = S + (b * a.L + tt) * a.ld_s;
        T* dst = sx + static_cast<int64_t>(r) * dp;
        for (int c = lane; c < dp; c += 64) dst[c] = (ok && c < D) ? src[c] : T(0);
      }
    }
  }
  __syncthreads();

  const int p = tid >> 4, g0 = tid & 15;
  const int64_t t = t0 + p;
  const bool tok = t < a.L;
  // 3. window scores, ternary decisions and their normalisation (ent_scores_kernel arithmetic)
  {
    const float sq = static_cast<float>(sqrt(static_cast<double>(a.R)));
    // float4 LDS reads need 16-byte aligned rows and halves: R % 8 == 0 (krs = R + 4)
    const int half4 = (half % 4 == 0) ? half : 0;
    float tern[4];  // W <= 64: slots w0, w0 + 16, ...
    float n = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = g0 + 16 * i;
      tern[i] = 0.0f;
      if (w >= W) continue;
      const int64_t j = t - (W - 1) + w;
      if (tok && j >= 0) {
        const float* qp = qr + p * krs;
        const float* kp = kr + (p + w) * krs;
        float dot = 0.0f;
        for (int c = 0; c < half4; c += 4) {
          const float4 qa = *reinterpret_cast<const float4*>(qp + c);
          const float4 ka = *reinterpret_cast<const float4*>(kp + c);
          const float4 qb = *reinterpret_cast<const float4*>(qp + half + c);
          const float4 kb = *reinterpret_cast<const float4*>(kp + half + c);
          dot = madd<DT>(qa.x, ka.x, dot);
          dot = madd<DT>(qb.x, kb.x, dot);
          dot = madd<DT>(qa.y, ka.y, dot);
          dot = madd<DT>(qb.y, kb.y, dot);
          dot = madd<DT>(qa.z, ka.z, dot);
          dot = madd<DT>(qb.z, kb.z, dot);
          dot = madd<DT>(qa.w, ka.w, dot);
          dot = madd<DT>(qb.w, kb.w, dot);
        }
        for (int c = half4; c < half; ++c) {
          dot = madd<DT>(qp[c], kp[c], dot);
          dot += qp[half + c] * kp[half + c];
        }
        float sc = rnd<DT>(rnd<DT>(dot) / sq);
        sc = rnd<DT>(sc + wbias[i]);
        tern[i] = sc > a.thr ? 1.0f : (sc < -a.thr ? -1.0f : 0.0f);
      }
      n += fabsf(tern[i]);
      if (a.tern && tok) a.tern[(b * a.L + t) * W + w] = static_cast<int8_t>(tern[i]);
    }
    n = wave_sum_f<16>(n);
    n = fmaxf(n, 1.0f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int w = g0 + 16 * i;
      if (w < W) wn[p * W + w] = rnd<DT>(tern[i] / n);
    }
  }
  __syncthreads();

  // 4. window sums, mix and tanh for the thread's channel groups (ent_mix_kernel arithmetic)
  const int groups = dp / 16;
  float tv[kFusedMaxGPT][16], cv[kFusedMaxGPT][16];
  float mx_t = 0.0f, mx_c = 0.0f;
#pragma unroll
  for (int gi = 0; gi < kFusedMaxGPT; ++gi) {
    const int g = g0 + 16 * gi;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      tv[gi][e] = 0.0f;
      cv[gi][e] = 0.0f;
    }
    if (g >= groups || !tok) continue;
    float acc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.0f;
    // four window rows' LDS reads in flight per step; each channel still sums w = 0, 1, .. in order
    int w = 0;
    for (; w + 4 <= W; w += 4) {
      float x[4][16], wt[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        lds_row16<DT>(sx + static_cast<int64_t>(p + w + u) * dp + 16 * g, x[u]);
        wt[u] = wn[p * W + w + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = madd<DT>(wt[u], x[u][e], acc[e]);
    }
    for (; w < W; ++w) {
      float x[16];
      lds_row16<DT>(sx + static_cast<int64_t>(p + w) * dp + 16 * g, x);
      const float wt = wn[p * W + w];
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[e] = madd<DT>(wt, x[e], acc[e]);
    }
    float sv[16];
    lds_row16<DT>(sx + static_cast<int64_t>(p + W - 1) * dp + 16 * g, sv);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int c = 16 * g + e;
      if (c >= D) continue;
      const float avg = rnd<DT>(acc[e]);
      const float s = sv[e];
      const float ev = rnd<DT>(s + rnd<DT>(a.ent_scale * rnd<DT>(avg - s)));
      cv[gi][e] = rnd<DT>(ev - s);
      tv[gi][e] = rnd<DT>(tanhf_(ev));
      mx_t = fmaxf(mx_t, fabsf(tv[gi][e]));
      mx_c = fmaxf(mx_c, fabsf(cv[gi][e]));
      if (a.e_tanh || a.c_out) {
        const int64_t o = (b * a.L + t) * a.ld_out + c;
        if (a.c_out) st<DT>(a.c_out, o, cv[gi][e]);
        if (a.e_tanh) st<DT>(a.e_tanh, o, tv[gi][e]);
      }
    }
  }
  // 5. per-token scales and codes (tesm.py:206-209); a position's 16 lanes share its row
  mx_t = wave_max<16>(mx_t);
  mx_c = wave_max<16>(mx_c);
  const float sc_t = act_scale<DT>(mx_t, a.eps);
  const float sc_c = act_scale<DT>(mx_c, a.eps);
  int sum_t = 0, sum_c = 0;
  const int64_t row = b * a.L + t;
  const int ngq = static_cast<int>(a.ldq / 16);
#pragma unroll
  for (int gi = 0; gi < kFusedMaxGPT; ++gi) {
    const int g = g0 + 16 * gi;
    if (!tok || g >= ngq) continue;
    uint32_t qt[16], qc[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const int c1 = (g < groups) ? act_code<DT>(tv[gi][e], sc_t) : 0;
      const int c2 = (g < groups) ? act_code<DT>(cv[gi][e], sc_c) : 0;
      sum_t += c1;
      sum_c += c2;
      qt[e] = static_cast<uint32_t>(c1) & 0xffu;
      qc[e] = static_cast<uint32_t>(c2) & 0xffu;
    }
    // layout 1: byte 4s + j of the group holds code 4j + s
    const uint4 ot = make_uint4(qt[0] | (qt[4] << 8) | (qt[8] << 16) | (qt[12] << 24),
                                qt[1] | (qt[5] << 8) | (qt[9] << 16) | (qt[13] << 24),
                                qt[2] | (qt[6] << 8) | (qt[10] << 16) | (qt[14] << 24),
                                qt[3] | (qt[7] << 8) | (qt[11] << 16) | (qt[15] << 24));
    const uint4 oc = make_uint4(qc[0] | (qc[4] << 8) | (qc[8] << 16) | (qc[12] << 24),
                                qc[1] | (qc[5] << 8) | (qc[9] << 16) | (qc[13] << 24),
                                qc[2] | (qc[6] << 8) | (qc[10] << 16) | (qc[14] << 24),
                                qc[3] | (qc[7] << 8) | (qc[11] << 16) | (qc[15] << 24));
    reinterpret_cast<uint4*>(a.q_te + row * a.ldq)[g] = ot;
    reinterpret_cast<uint4*>(a.q_c + row * a.ldq)[g] = oc;
  }
  // code groups of the padding past the thread's range (ldq > 512) are zero as well
  for (int g = g0 + 16 * kFusedMaxGPT; tok && g < ngq; g += 16) {
    reinterpret_cast<uint4*>(a.q_te + row * a.ldq)[g] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(a.q_c + row * a.ldq)[g] = make_uint4(0, 0, 0, 0);
  }
  sum_t = wave_sum_i<16>(sum_t);
  sum_c = wave_sum_i<16>(sum_c);
  if (tok && g0 == 0) {
    a.s_te[row] = sc_t;
    a.rs_te[row] = sum_t;
    a.s_c[row] = sc_c;
    a.rs_c[row] = sum_c;
  }
}

// Fused SISO kernel, second form: 32 threads per position, each owning an 8-channel slice (D <= 512,
// D % 8 == 0), 16 positions per workgroup of 512 threads -- twice the waves of ent_fused_kernel on the
// same work.  The state halo is converted to float32 once while it is staged (instead of once per
// window row that reads it), in chunk order (q, s): the 16-byte half q of slice s at chunk
// q * nsl + s, so the 16 lanes of a read pass take 256 contiguous bytes.  The arithmetic and its
// order are ent_fused_kernel's, so the two give the same bits.  Layout-1 codes of a 16-channel group
// come from a lane pair (slices 2g, 2g + 1): each lane forms its two bytes of every dword, the pair
// swaps them, the even lane stores the group.
constexpr int kF2TP = 16;
constexpr int kF2TPP = 32;
constexpr int kF2MaxSPT = 2;

struct Fused2Lds {
  int64_t kr, qr, wn, sx, total;  // byte offsets
  int64_t krs;                    // row stride of kr / qr in floats
  int64_t nsl;                    // 8-channel slices per row
};

__host__ __device__ inline Fused2Lds fused2_lds(int64_t R, int64_t D, int64_t weff) {
  Fused2Lds f;
  const int64_t rows = kF2TP + weff - 1;
  f.krs = R + 4;
  f.nsl = D / 8;
  f.kr = 0;
  f.qr = f.kr + rows * f.krs * 4;
  f.wn = f.qr + kF2TP * f.krs * 4;
  f.sx = (f.wn + kF2TP * weff * 4 + 15) / 16 * 16;
  f.total = f.sx + rows * f.nsl * 32;
  return f;
}

// Stores of a thread's 8 consecutive channels of one output: two 4-wide stores when the row and base allow.
template <int DT>
__device__ __forceinline__ void st8(void* p, int64_t o, const float (&v)[8], bool vec) {
  if (vec) {
    const float lo[4] = {v[0], v[1], v[2], v[3]}, hi[4] = {v[4], v[5], v[6], v[7]};
    st4<DT>(p, o, lo);
    st4<DT>(p, o + 4, hi);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) st<DT>(p, o + e, v[e]);
  }
}

// QUANT: the layer's form (int8 codes of tanh(E) and C, optionally their float values too); otherwise
// the float outputs alone (window average, E, tanh(E), C; each optional), as the unfused kernels give them.
// KI: staging items per thread for the states and keys (the queries take KI / 2), 2 where the rows fit
// (every item slot issues a load, so unused slots cost memory instructions), else 4.
template <int DT, bool QUANT, int KI>
__global__ __launch_bounds__(512) void ent_fused2_kernel(EntArgs a, int64_t weff, Fused2Lds f) {
  using T = typename Elem<DT>::T;
  extern __shared__ __attribute__((aligned(16))) char lds_f2[];
  float* kr = reinterpret_cast<float*>(lds_f2 + f.kr);
  float* qr = reinterpret_cast<float*>(lds_f2 + f.qr);
  float* wn = reinterpret_cast<float*>(lds_f2 + f.wn);
  float* sx = reinterpret_cast<float*>(lds_f2 + f.sx);
  const int tid = threadIdx.x;
  __builtin_assume(tid < 512);
  const int64_t b = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kF2TP;
  const int half = static_cast<int>(a.R / 2), D = static_cast<int>(a.D), W = static_cast<int>(weff);
  const int krs = static_cast<int>(f.krs), nsl = static_cast<int>(f.nsl);
  const int rows = kF2TP + W - 1;
  const int64_t tk0 = t0 - (W - 1);  // position of key row 0
  const int p = tid / kF2TPP, h8 = tid % kF2TPP;

  // window bias of the thread's score slots w = h8, h8 + 32 (read first, used after the LDS phase)
  float wbias[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int w = h8 + 32 * i;
    wbias[i] = a.bias[a.W - W + (w < W ? w : W - 1)];
  }

  // 1. staging: keys and queries RoPE'd into float32 rows, the state halo converted to float32.  All of
  //    a thread's loads are requested before any is used; rows outside [0, L) are zero.
  const T* S = static_cast<const T*>(a.S);
  {
    constexpr int kSI = KI, kKI = KI, kQI = KI / 2;  // items per thread (checked on the host)
    v4i sv[kSI][DT == kBF16 ? 1 : 2];
    int sr[kSI], ss[kSI];
#pragma unroll
    for (int k = 0; k < kSI; ++k) {
      const int i = tid + 512 * k;
      const int r = i / nsl, sl = i - r * nsl;
      sr[k] = r;
      ss[k] = sl;
      int64_t tt = tk0 + (r < rows ? r : rows - 1);
      tt = tt < 0 ? 0 : (tt >= a.L ? a.L - 1 : tt);
      const T* src = S + (b * a.L + tt) * a.ld_s + 8 * sl;
      sv[k][0] = *reinterpret_cast<const v4i*>(src);
      if constexpr (DT != kBF16) sv[k][1] = *reinterpret_cast<const v4i*>(src + 4);
    }
    float kxa[kKI], kxb[kKI], qxa[kQI], qxb[kQI], qaa[kQI], qab[kQI];
    float2 kcs[kKI], qcs[kQI];
#pragma unroll
    for (int k = 0; k < kKI; ++k) {
      const int i = tid + 512 * k;
      const int r = i / half, c = i - r * half;
      int64_t tt = tk0 + (r < rows ? r : rows - 1);
      tt = tt < 0 ? 0 : (tt >= a.L ? a.L - 1 : tt);
      const int64_t ko = (b * a.L + tt) * a.ld_k;
      kxa[k] = ld<DT>(a.k, ko + c);
      kxb[k] = ld<DT>(a.k, ko + half + c);
      kcs[k] = a.rope[tt * half + c];
    }
#pragma unroll
    for (int k = 0; k < kQI; ++k) {
      const int i = tid + 512 * k;
      const int pp = i / half, c = i - pp * half;
      const int64_t tt = (t0 + pp < a.L) ? t0 + pp : a.L - 1;
      const int64_t qo = (b * a.L + tt) * a.ld_q;
      qxa[k] = ld<DT>(a.q, qo + c);
      qxb[k] = ld<DT>(a.q, qo + half + c);
      qcs[k] = a.rope[tt * half + c];
      qaa[k] = qab[k] = 0.0f;
      if (a.q_add) {
        const int64_t ao = (b * a.L + tt) * a.ld_qadd;
        qaa[k] = ld<DT>(a.q_add, ao + c);
        qab[k] = ld<DT>(a.q_add, ao + half + c);
      }
    }
#pragma unroll
    for (int k = 0; k < kSI; ++k) {
      const int r = sr[k];
      if (r >= rows) break;
      const int64_t tt = tk0 + r;
      const bool ok = tt >= 0 && tt < a.L;
      float x[8];
      if constexpr (DT == kBF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wd = static_cast<uint32_t>(sv[k][0][i]);
          x[2 * i] = ok ? __uint_as_float(wd << 16) : 0.0f;
          x[2 * i + 1] = ok ? __uint_as_float(wd & 0xffff0000u) : 0.0f;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = ok ? __int_as_float(sv[k][i >> 2][i & 3]) : 0.0f;
      }
      float* row = sx + static_cast<int64_t>(r) * nsl * 8;
      *reinterpret_cast<float4*>(row + 4 * ss[k]) = make_float4(x[0], x[1], x[2], x[3]);
      *reinterpret_cast<float4*>(row + 4 * (nsl + ss[k])) = make_float4(x[4], x[5], x[6], x[7]);
    }
#pragma unroll
    for (int k = 0; k < kKI; ++k) {
      const int i = tid + 512 * k;
      const int r = i / half, c = i - r * half;
      if (r >= rows) break;
      const int64_t tt = tk0 + r;
      float o1 = 0.0f, o2 = 0.0f;
      if (tt >= 0 && tt < a.L) rope_pair<DT>(kxa[k], kxb[k], kcs[k], o1, o2);
      kr[r * krs + c] = o1;
      kr[r * krs + half + c] = o2;
    }
#pragma unroll
    for (int k = 0; k < kQI; ++k) {
      const int i = tid + 512 * k;
      const int pp = i / half, c = i - pp * half;
      if (pp >= kF2TP) break;
      float o1 = 0.0f, o2 = 0.0f;
      if (t0 + pp < a.L) {
        rope_pair<DT>(qxa[k], qxb[k], qcs[k], o1, o2);
        if (a.q_add) {
          o1 = rnd<DT>(o1 + qaa[k]);
          o2 = rnd<DT>(o2 + qab[k]);
        }
      }
      qr[pp * krs + c] = o1;
      qr[pp * krs + half + c] = o2;
    }
  }
  __syncthreads();

  const int64_t t = t0 + p;
  const bool tok = t < a.L;
  // 2. window scores, ternary decisions and their normalisation (ent_fused_kernel's arithmetic)
  {
    const float sq = static_cast<float>(sqrt(static_cast<double>(a.R)));
    const int half4 = (half % 4 == 0) ? half : 0;
    float tern[2];
    float n = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int w = h8 + 32 * i;
      tern[i] = 0.0f;
      if (w >= W) continue;
      const int64_t j = t - (W - 1) + w;
      if (tok && j >= 0) {
        const float* qp = qr + p * krs;
        const float* kp = kr + (p + w) * krs;
        float dot = 0.0f;
        for (int c = 0; c < half4; c += 4) {
          const float4 qa = *reinterpret_cast<const float4*>(qp + c);
          const float4 ka = *reinterpret_cast<const float4*>(kp + c);
          const float4 qb = *reinterpret_cast<const float4*>(qp + half + c);
          const float4 kb = *reinterpret_cast<const float4*>(kp + half + c);
          dot = madd<DT>(qa.x, ka.x, dot);
          dot = madd<DT>(qb.x, kb.x, dot);
          dot = madd<DT>(qa.y, ka.y, dot);
          dot = madd<DT>(qb.y, kb.y, dot);
          dot = madd<DT>(qa.z, ka.z, dot);
          dot = madd<DT>(qb.z, kb.z, dot);
          dot = madd<DT>(qa.w, ka.w, dot);
          dot = madd<DT>(qb.w, kb.w, dot);
        }
        for (int c = half4; c < half; ++c) {
          dot = madd<DT>(qp[c], kp[c], dot);
          dot += qp[half + c] * kp[half + c];
        }
        float sc = rnd<DT>(rnd<DT>(dot) / sq);
        sc = rnd<DT>(sc + wbias[i]);
        tern[i] = sc > a.thr ? 1.0f : (sc < -a.thr ? -1.0f : 0.0f);
      }
      n += fabsf(tern[i]);
      if (a.tern && tok) a.tern[(b * a.L + t) * W + w] = static_cast<int8_t>(tern[i]);
    }
    n = static_cast<float>(wave_sum_i<kF2TPP>(static_cast<int>(n)));  // a count: exact in any order
    n = fmaxf(n, 1.0f);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int w = h8 + 32 * i;
      if (w < W) wn[p * W + w] = rnd<DT>(tern[i] / n);
    }
  }
  __syncthreads();

  // 3. window sums, mix and tanh of the thread's slices
  // 4-wide output stores when every requested output is 4-element aligned and rows are 4 elements apart
  constexpr uintptr_t kAl = DT == kBF16 ? 8 : 16;
  const bool vout = a.ld_out % 4 == 0 && reinterpret_cast<uintptr_t>(a.avg) % kAl == 0 &&
                    reinterpret_cast<uintptr_t>(a.e_out) % kAl == 0 && reinterpret_cast<uintptr_t>(a.e_tanh) % kAl == 0 &&
                    reinterpret_cast<uintptr_t>(a.c_out) % kAl == 0;
  float tv[kF2MaxSPT][8], cv[kF2MaxSPT][8];
  float mx_t = 0.0f, mx_c = 0.0f;
#pragma unroll
  for (int si = 0; si < kF2MaxSPT; ++si) {
    const int sl = h8 + kF2TPP * si;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      tv[si][e] = 0.0f;
      cv[si][e] = 0.0f;
    }
    if (sl >= nsl || !tok) continue;
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    auto row8 = [&](int r, float (&x)[8]) {
      const float* rp = sx + static_cast<int64_t>(r) * nsl * 8;
      const float4 lo = *reinterpret_cast<const float4*>(rp + 4 * sl);
      const float4 hi = *reinterpret_cast<const float4*>(rp + 4 * (nsl + sl));
      x[0] = lo.x, x[1] = lo.y, x[2] = lo.z, x[3] = lo.w, x[4] = hi.x, x[5] = hi.y, x[6] = hi.z, x[7] = hi.w;
    };
    int w = 0;
    for (; w + 4 <= W; w += 4) {  // four rows' reads in flight; each channel sums w = 0, 1, .. in order
      float x[4][8], wt[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        row8(p + w + u, x[u]);
        wt[u] = wn[p * W + w + u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] = madd<DT>(wt[u], x[u][e], acc[e]);
    }
    for (; w < W; ++w) {
      float x[8];
      row8(p + w, x);
      const float wt = wn[p * W + w];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = madd<DT>(wt, x[e], acc[e]);
    }
    float sv[8], av[8], evs[8];
    row8(p + W - 1, sv);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float avg = rnd<DT>(acc[e]);
      const float s0 = sv[e];
      const float ev = rnd<DT>(s0 + rnd<DT>(a.ent_scale * rnd<DT>(avg - s0)));
      av[e] = avg;
      evs[e] = ev;
      cv[si][e] = rnd<DT>(ev - s0);
      tv[si][e] = rnd<DT>(tanhf_(ev));
      mx_t = fmaxf(mx_t, fabsf(tv[si][e]));
      mx_c = fmaxf(mx_c, fabsf(cv[si][e]));
    }
    if (a.e_tanh || a.c_out || a.avg || a.e_out) {
      const int64_t o = (b * a.L + t) * a.ld_out + 8 * sl;
      if (a.c_out) st8<DT>(a.c_out, o, cv[si], vout);
      if (a.e_tanh) st8<DT>(a.e_tanh, o, tv[si], vout);
      if (a.avg) st8<DT>(a.avg, o, av, vout);
      if (a.e_out) st8<DT>(a.e_out, o, evs, vout);
    }
  }
  if constexpr (!QUANT) return;
  // 4. per-token scales and codes (tesm.py:206-209); a position's 32 lanes share its row
  mx_t = wave_max<kF2TPP>(mx_t);
  mx_c = wave_max<kF2TPP>(mx_c);
  const float sc_t = act_scale<DT>(mx_t, a.eps);
  const float sc_c = act_scale<DT>(mx_c, a.eps);
  int sum_t = 0, sum_c = 0;
  const int64_t row = b * a.L + t;
  const int ngq = static_cast<int>(a.ldq / 16), groups = D / 16;
#pragma unroll
  for (int si = 0; si < kF2MaxSPT; ++si) {
    const int sl = h8 + kF2TPP * si, g = sl >> 1, hh = sl & 1;
    if (2 * (kF2TPP * si) >= 2 * nsl) break;  // no thread of this round has a slice (uniform)
    // layout 1: byte 4s + j of the group holds code 4j + s; this lane's codes e = 8 hh + i sit at
    // bytes 4 (i & 3) + 2 hh + (i >> 2)
    uint32_t pt[4] = {0, 0, 0, 0}, pc[4] = {0, 0, 0, 0};
    if (sl < nsl && tok) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c1 = act_code<DT>(tv[si][i], sc_t), c2 = act_code<DT>(cv[si][i], sc_c);
        sum_t += c1;
        sum_c += c2;
        const int sh = 8 * (2 * hh + (i >> 2));
        pt[i & 3] |= (static_cast<uint32_t>(c1) & 0xffu) << sh;
        pc[i & 3] |= (static_cast<uint32_t>(c2) & 0xffu) << sh;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      pt[q] |= static_cast<uint32_t>(dpp_mov<kDppXor1>(static_cast<int>(pt[q])));  // lane ^ 1
      pc[q] |= static_cast<uint32_t>(dpp_mov<kDppXor1>(static_cast<int>(pc[q])));
    }
    if (tok && hh == 0 && g < ngq) {
      reinterpret_cast<uint4*>(a.q_te + row * a.ldq)[g] = make_uint4(pt[0], pt[1], pt[2], pt[3]);
      reinterpret_cast<uint4*>(a.q_c + row * a.ldq)[g] = make_uint4(pc[0], pc[1], pc[2], pc[3]);
    }
  }
  // code groups of the padding (ldq > D) are zero
  for (int g = groups + h8; tok && g < ngq; g += kF2TPP) {
    reinterpret_cast<uint4*>(a.q_te + row * a.ldq)[g] = make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(a.q_c + row * a.ldq)[g] = make_uint4(0, 0, 0, 0);
  }
  sum_t = wave_sum_i<kF2TPP>(sum_t);
  sum_c = wave_sum_i<kF2TPP>(sum_c);
  if (tok && h8 == 0) {
    a.s_te[row] = sc_t;
    a.rs_te[row] = sum_t;
    a.s_c[row] = sc_c;
    a.rs_c[row] = sum_c;
  }
}

// ---------------------------------------------------------------------------
// Fused SISO kernel, third form: the window mix in registers, for the shapes whose state halo does not
// fit ent_fused2_kernel's LDS (D 384-512 with window 32; D 384 with rank 96).  A workgroup owns (batch
// row b, 2 TS positions) and all D channels (D % 64 == 0, D <= 512); thread (s, ch) owns channel ch of
// the TS positions of half s.  A position's window mix reads its own channel's states only, so the thread
// loads the W - 1 + 16 states of its channel it needs (as raw bits, all in flight at once, straight
// from the state tensor) and forms its 16 window sums from registers, the window weights being the
// same for all 64 lanes of a wave (broadcast LDS reads).  The weights come from one (position, window
// slot) pair per thread over RoPE'd q / k rows staged in LDS; tanh(E) and C are staged in LDS and
// quantized with one 16-channel group per thread.  Every value is the same sequence of float
// operations as in ent_fused2_kernel, so the two give the same bits.
// ---------------------------------------------------------------------------

struct RegLds {
  int64_t kr, qr, wn, stg, total;  // byte offsets
  int64_t krs;                     // row pitch of the RoPE'd key / query rows, floats
  int64_t nq;                      // quantities (tanh(E), C) staged per quantization pass
};

__host__ __device__ inline RegLds reg_lds(int64_t D, int64_t R, int64_t W, int wm, int es, int64_t tp) {
  auto al = [](int64_t v) { return (v + 15) / 16 * 16; };
  RegLds f;
  f.krs = R + 4;
  f.kr = 0;
  f.qr = al(f.kr + (tp + W - 1) * f.krs * 4);
  f.wn = al(f.qr + tp * f.krs * 4);
  const int64_t end_wn = f.wn + tp * wm * 4;
  // tanh(E) / C staging reuses the key rows onward once the mix has read the weights: both at once
  // where that stays within 64 KB
  f.stg = 0;
  const int64_t e1 = tp * D * es, e2 = 2 * e1;
  f.nq = (e2 <= end_wn || e2 <= 64 * 1024) ? 2 : 1;
  const int64_t end_stg = f.nq == 2 ? e2 : e1;
  f.total = end_wn > end_stg ? end_wn : end_stg;
  return f;
}

// WM: window slots of the mix (16 or 32; a window W < WM is right-aligned, the first WM - W slots
// weigh zero).  KI: key staging items per thread in the first round (queries: 2).
template <int DT, int WM, int KI, int NTM, int TS>
__global__ __launch_bounds__(NTM, 1) void ent_reg_kernel(EntArgs e, int64_t weff, RegLds f) {
  using T = typename Elem<DT>::T;
  constexpr int TP = 2 * TS, NX = WM - 1 + TS;
  extern __shared__ __attribute__((aligned(16))) char lds_rg[];
  float* kr = reinterpret_cast<float*>(lds_rg + f.kr);
  float* qr = reinterpret_cast<float*>(lds_rg + f.qr);
  float* wn = reinterpret_cast<float*>(lds_rg + f.wn);
  T* stg = reinterpret_cast<T*>(lds_rg + f.stg);
  const int tid = threadIdx.x;
  const int D = static_cast<int>(e.D), W = static_cast<int>(weff), half = static_cast<int>(e.R / 2);
  const int krs = static_cast<int>(f.krs), NT = 2 * D;
  const int s = __builtin_amdgcn_readfirstlane(tid / D);  // D % 64 == 0: uniform per wave
  const int ch = tid - s * D;
  const int64_t L = e.L, b = blockIdx.y;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * TP, ts = t0 + s * TS;
  const int n = ts >= L ? 0 : static_cast<int>(ts + TS < L ? TS : L - ts);  // wave-uniform
  const int rows = TP + W - 1;
  const int64_t tk0 = t0 - (W - 1);
  const int zs = WM - W;  // leading zero-weight slots

  // 1. every load: the states of the thread's window rows (x[k] is position ts - (WM - 1) + k; rows
  //    outside [0, L) and the zero-weight slots re-read a valid row and are zeroed), keys and queries
  //    with their RoPE rows, the window bias of the thread's first score slot
  uint32_t xb[NX];
  {
    const T* S = static_cast<const T*>(e.S);
#pragma unroll
    for (int k = 0; k < NX; ++k) {
      int64_t pos = ts - (WM - 1) + k;
      pos = pos < 0 ? 0 : (pos >= L ? L - 1 : pos);
      xb[k] = ld_bits<DT>(S + (b * L + pos) * e.ld_s, ch);
    }
  }
  constexpr int kQI = 2;
  float kxa[KI], kxb[KI], qxa[kQI], qxb[kQI], qaa[kQI], qab[kQI];
  float2 kcs[KI], qcs[kQI];
#pragma unroll
  for (int k = 0; k < KI; ++k) {
    const int i = tid + NT * k;
    const int r = i / half, cc = i - r * half;
    int64_t tt = tk0 + (r < rows ? r : rows - 1);
    tt = tt < 0 ? 0 : (tt >= L ? L - 1 : tt);
    const int64_t ko = (b * L + tt) * e.ld_k;
    kxa[k] = ld<DT>(e.k, ko + cc);
    kxb[k] = ld<DT>(e.k, ko + half + cc);
    kcs[k] = e.rope[tt * half + cc];
  }
#pragma unroll
  for (int k = 0; k < kQI; ++k) {
    const int i = tid + NT * k;
    const int pp = i / half, cc = i - pp * half;
    const int64_t tt = (t0 + pp < L && pp < TP) ? t0 + pp : L - 1;
    const int64_t qo = (b * L + tt) * e.ld_q;
    qxa[k] = ld<DT>(e.q, qo + cc);
    qxb[k] = ld<DT>(e.q, qo + half + cc);
    qcs[k] = e.rope[tt * half + cc];
    qaa[k] = qab[k] = 0.0f;
    if (e.q_add) {
      const int64_t ao = (b * L + tt) * e.ld_qadd;
      qaa[k] = ld<DT>(e.q_add, ao + cc);
      qab[k] = ld<DT>(e.q_add, ao + half + cc);
    }
  }
  float wbias0;
  {
    const int w = tid % WM;
    wbias0 = e.bias[e.W - W + (w < W ? w : W - 1)];
  }

  // 2. RoPE'd keys and queries into LDS (rows outside [0, L) are zero); items beyond the first round
  //    (small D with a wide rank) are loaded and rotated one at a time
#pragma unroll
  for (int k = 0; k < KI; ++k) {
    const int i = tid + NT * k;
    const int r = i / half, cc = i - r * half;
    if (r >= rows) break;
    const int64_t tt = tk0 + r;
    float o1 = 0.0f, o2 = 0.0f;
    if (tt >= 0 && tt < L) rope_pair<DT>(kxa[k], kxb[k], kcs[k], o1, o2);
    kr[r * krs + cc] = o1;
    kr[r * krs + half + cc] = o2;
  }
#pragma unroll
  for (int k = 0; k < kQI; ++k) {
    const int i = tid + NT * k;
    const int pp = i / half, cc = i - pp * half;
    if (pp >= TP) break;
    float o1 = 0.0f, o2 = 0.0f;
    if (t0 + pp < L) {
      rope_pair<DT>(qxa[k], qxb[k], qcs[k], o1, o2);
      if (e.q_add) {
        o1 = rnd<DT>(o1 + qaa[k]);
        o2 = rnd<DT>(o2 + qab[k]);
      }
    }
    qr[pp * krs + cc] = o1;
    qr[pp * krs + half + cc] = o2;
  }
  for (int i = tid + NT * KI; i < rows * half; i += NT) {
    const int r = i / half, cc = i - r * half;
    const int64_t tt = tk0 + r;
    float o1 = 0.0f, o2 = 0.0f;
    if (tt >= 0 && tt < L) {
      const int64_t ko = (b * L + tt) * e.ld_k;
      rope_pair<DT>(ld<DT>(e.k, ko + cc), ld<DT>(e.k, ko + half + cc), e.rope[tt * half + cc], o1, o2);
    }
    kr[r * krs + cc] = o1;
    kr[r * krs + half + cc] = o2;
  }
  for (int i = tid + NT * kQI; i < TP * half; i += NT) {
    const int pp = i / half, cc = i - pp * half;
    const int64_t tt = t0 + pp;
    float o1 = 0.0f, o2 = 0.0f;
    if (tt < L) {
      const int64_t qo = (b * L + tt) * e.ld_q;
      rope_pair<DT>(ld<DT>(e.q, qo + cc), ld<DT>(e.q, qo + half + cc), e.rope[tt * half + cc], o1, o2);
      if (e.q_add) {
        const int64_t ao = (b * L + tt) * e.ld_qadd;
        o1 = rnd<DT>(o1 + ld<DT>(e.q_add, ao + cc));
        o2 = rnd<DT>(o2 + ld<DT>(e.q_add, ao + half + cc));
      }
    }
    qr[pp * krs + cc] = o1;
    qr[pp * krs + half + cc] = o2;
  }
  __syncthreads();

  // 3. window scores, ternary decisions and weights (ent_fused2_kernel's arithmetic); WM lanes per
  //    position, slot w of the effective window at weight column WM - W + w
  {
    const float sq = static_cast<float>(sqrt(static_cast<double>(e.R)));
    const int half4 = (half % 4 == 0) ? half : 0;
    for (int item = tid; item < TP * WM; item += NT) {  // uniform per wave (TP * WM, NT multiples of 64)
      const int p = item / WM, w = item % WM;
      const int64_t t = t0 + p;
      const bool tok = t < L;
      float tern = 0.0f;
      if (w < W) {
        const int64_t j = t - (W - 1) + w;
        if (tok && j >= 0) {
          const float* qp = qr + p * krs;
          const float* kp = kr + (p + w) * krs;
          float dot = 0.0f;
          for (int cc = 0; cc < half4; cc += 4) {
            const float4 qa = *reinterpret_cast<const float4*>(qp + cc);
            const float4 ka = *reinterpret_cast<const float4*>(kp + cc);
            const float4 qb = *reinterpret_cast<const float4*>(qp + half + cc);
            const float4 kb = *reinterpret_cast<const float4*>(kp + half + cc);
            dot = madd<DT>(qa.x, ka.x, dot);
            dot = madd<DT>(qb.x, kb.x, dot);
            dot = madd<DT>(qa.y, ka.y, dot);
            dot = madd<DT>(qb.y, kb.y, dot);
            dot = madd<DT>(qa.z, ka.z, dot);
            dot = madd<DT>(qb.z, kb.z, dot);
            dot = madd<DT>(qa.w, ka.w, dot);
            dot = madd<DT>(qb.w, kb.w, dot);
          }
          for (int cc = half4; cc < half; ++cc) {
            dot = madd<DT>(qp[cc], kp[cc], dot);
            dot = madd<DT>(qp[half + cc], kp[half + cc], dot);
          }
          float sc = rnd<DT>(rnd<DT>(dot) / sq);
          const float wb = item == tid ? wbias0 : e.bias[e.W - W + w];
          sc = rnd<DT>(sc + wb);
          tern = sc > e.thr ? 1.0f : (sc < -e.thr ? -1.0f : 0.0f);
        }
        if (e.tern && tok) e.tern[(b * L + t) * W + w] = static_cast<int8_t>(tern);
      }
      float nn = static_cast<float>(wave_sum_i<WM>(static_cast<int>(fabsf(tern))));  // a count: exact
      nn = fmaxf(nn, 1.0f);
      if (w < W)
        wn[p * WM + (WM - W) + w] = rnd<DT>(tern / nn);
      else
        wn[p * WM + (w - W)] = 0.0f;
    }
  }
  __syncthreads();

  // 4. window sums of the thread's TS positions (slots in order, as ent_fused2_kernel sums them), E,
  //    tanh(E) and C
  float x[NX];
#pragma unroll
  for (int k = 0; k < NX; ++k) {
    const int64_t pos = ts - (WM - 1) + k;
    const bool in = k >= zs && pos >= 0 && pos < L;
    x[k] = in ? from_bits<DT>(xb[k]) : 0.0f;
  }
  float tv[TS], cv[TS];
  {
    float acc[TS];
#pragma unroll
    for (int i = 0; i < TS; ++i) acc[i] = 0.0f;
#pragma unroll
    for (int w4 = 0; w4 < WM; w4 += 4) {
#pragma unroll
      for (int i = 0; i < TS; ++i) {
        const float4 wt = *reinterpret_cast<const float4*>(wn + (s * TS + i) * WM + w4);
        acc[i] = madd<DT>(wt.x, x[i + w4], acc[i]);
        acc[i] = madd<DT>(wt.y, x[i + w4 + 1], acc[i]);
        acc[i] = madd<DT>(wt.z, x[i + w4 + 2], acc[i]);
        acc[i] = madd<DT>(wt.w, x[i + w4 + 3], acc[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < TS; ++i) {
      const float s0 = x[WM - 1 + i];
      const float avg = rnd<DT>(acc[i]);
      const float ev = rnd<DT>(s0 + rnd<DT>(e.ent_scale * rnd<DT>(avg - s0)));
      cv[i] = rnd<DT>(ev - s0);
      tv[i] = rnd<DT>(tanhf_(ev));
    }
  }
  if (e.e_tanh || e.c_out) {
#pragma unroll
    for (int i = 0; i < TS; ++i) {
      if (i >= n) break;
      const int64_t o = (b * L + ts + i) * e.ld_out + ch;
      if (e.e_tanh) st<DT>(e.e_tanh, o, tv[i]);
      if (e.c_out) st<DT>(e.c_out, o, cv[i]);
    }
  }

  // 5. per-token codes of tanh(E) and of C: each thread's column staged in LDS (both quantities in one
  //    pass where they fit, f.nq = 2, else one at a time), then one 16-channel group per thread, GQ
  //    lanes per position (a power of two >= D / 16)
  const int groups = D / 16, ngq = static_cast<int>(e.ldq / 16);
  const int GQ = groups <= 4 ? 4 : (groups <= 8 ? 8 : (groups <= 16 ? 16 : 32));
  const int nq = static_cast<int>(f.nq);
  constexpr int NV = 16 * static_cast<int>(sizeof(T)) / 16;  // 16-byte LDS reads per group
  for (int q0 = 0; q0 < 2; q0 += nq) {
    __syncthreads();  // the mix's (or the previous pass's) LDS reads are done
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      if (q < q0 || q >= q0 + nq) continue;  // uniform
      T* row0 = stg + ((q - q0) * TP + s * TS) * D + ch;
#pragma unroll
      for (int i = 0; i < TS; ++i) {
        const float v = q == 0 ? tv[i] : cv[i];
        if constexpr (DT == kBF16)
          row0[i * D] = static_cast<T>(__float_as_uint(v) >> 16);
        else
          row0[i * D] = v;
      }
    }
    __syncthreads();
    for (int item = tid; item < nq * TP * GQ; item += NT) {  // uniform per wave (TP * GQ % 64 == 0)
      const int ql = item / (TP * GQ), rem = item - ql * (TP * GQ), qn = q0 + ql;
      const int p = rem / GQ, gi = rem % GQ;
      const int64_t t = t0 + p, row = b * L + t;
      const bool tok = t < L;
      int8_t* qo = qn == 0 ? e.q_te : e.q_c;
      float* so = qn == 0 ? e.s_te : e.s_c;
      int32_t* ro = qn == 0 ? e.rs_te : e.rs_c;
      const int gl = gi < groups ? gi : groups - 1;
      const uint4* src = reinterpret_cast<const uint4*>(stg + (ql * TP + p) * D + 16 * gl);
      uint4 raw[NV];
#pragma unroll
      for (int j = 0; j < NV; ++j) raw[j] = src[j];
      const uint32_t* wd = reinterpret_cast<const uint32_t*>(raw);
      float v[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float fv;
        if constexpr (DT == kBF16)
          fv = __uint_as_float(j % 2 == 0 ? wd[j / 2] << 16 : wd[j / 2] & 0xffff0000u);
        else
          fv = __uint_as_float(wd[j]);
        v[j] = gi < groups ? fv : 0.0f;
      }
      float mx = 0.0f;
#pragma unroll
      for (int j = 0; j < 16; ++j) mx = fmaxf(mx, fabsf(v[j]));
      if (GQ == 4) mx = wave_max<4>(mx);
      else if (GQ == 8) mx = wave_max<8>(mx);
      else if (GQ == 16) mx = wave_max<16>(mx);
      else mx = wave_max<32>(mx);
      const float sc = act_scale<DT>(mx, e.eps);
      int32_t rs = 0;
      const uint4 cw = group_codes<DT>(v, sc, 1, rs);
      if (tok && gi < groups) reinterpret_cast<uint4*>(qo + row * e.ldq)[gi] = cw;
      for (int gp = groups + gi; tok && gp < ngq; gp += GQ)
        reinterpret_cast<uint4*>(qo + row * e.ldq)[gp] = make_uint4(0, 0, 0, 0);
      if (GQ == 4) rs = wave_sum_i<4>(rs);
      else if (GQ == 8) rs = wave_sum_i<8>(rs);
      else if (GQ == 16) rs = wave_sum_i<16>(rs);
      else rs = wave_sum_i<32>(rs);
      if (tok && gi == 0) {
        so[row] = sc;
        ro[row] = rs;
      }
    }
  }
}

template <int DT, int MIMO>
int run_scores(const EntArgs& a, int64_t weff, hipStream_t st) {
  if (MIMO && a.q_add == nullptr) {
    const size_t lds = static_cast<size_t>((kScTP + kScTP + a.W - 1) * kScPitch) * sizeof(float);
    dim3 grid(static_cast<unsigned>((a.L + kScTP - 1) / kScTP), static_cast<unsigned>(a.B * a.H));
    ent_scores_mimo_kernel<DT><<<grid, 256, lds, TESM_LOGGED(st, ent_scores_mimo_kernel<DT>)>>>(a);
    return check_launch("entanglement scores (MIMO, tiled)");
  }
  const int64_t groups = a.B * a.L * a.H;
  auto blocks = [&](int wp) { return static_cast<unsigned>((groups * wp + 255) / 256); };
  if (weff <= 8) ent_scores_kernel<DT, MIMO, 8><<<blocks(8), 256, 0, TESM_LOGGED(st, ent_scores_kernel<DT, MIMO, 8>)>>>(a, weff, 0.f);
  else if (weff <= 16) ent_scores_kernel<DT, MIMO, 16><<<blocks(16), 256, 0, TESM_LOGGED(st, ent_scores_kernel<DT, MIMO, 16>)>>>(a, weff, 0.f);
  else if (weff <= 32) ent_scores_kernel<DT, MIMO, 32><<<blocks(32), 256, 0, TESM_LOGGED(st, ent_scores_kernel<DT, MIMO, 32>)>>>(a, weff, 0.f);
  else ent_scores_kernel<DT, MIMO, 64><<<blocks(64), 256, 0, TESM_LOGGED(st, ent_scores_kernel<DT, MIMO, 64>)>>>(a, weff, 0.f);
  return check_launch("entanglement scores");
}

template <int DT>
int run_mix(const EntArgs& a, int64_t weff, hipStream_t st) {
  dim3 grid(static_cast<unsigned>((a.D + kMixDS - 1) / kMixDS), static_cast<unsigned>((a.L + kMixTP - 1) / kMixTP),
            static_cast<unsigned>(a.B * a.H));
  const size_t lds = static_cast<size_t>((kMixTP + weff - 1) * kMixDS + kMixTP * weff) * sizeof(float);
  ent_mix_kernel<DT><<<grid, 256, lds, TESM_LOGGED(st, ent_mix_kernel<DT>)>>>(a, weff);
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
    rope_table_kernel<kBF16><<<nb, 256, 0, TESM_LOGGED(st, rope_table_kernel<kBF16>)>>>(tab, L, R, pos_offset, base);
  else
    rope_table_kernel<kF32><<<nb, 256, 0, TESM_LOGGED(st, rope_table_kernel<kF32>)>>>(tab, L, R, pos_offset, base);
  return check_launch("rope_table");
}

static int64_t eff_window(const EntArgs& a) { return a.mimo ? a.W : std::min(a.W, a.L); }

constexpr int kRegTS = 8;  // positions per thread of the register-mix kernel (16 per workgroup)

template <int DT, int WM, int KI>
static void launch_reg_k(const EntArgs& a, int64_t weff, const RegLds& f, hipStream_t st) {
  constexpr int TS = kRegTS;
  dim3 grid(static_cast<unsigned>((a.L + 2 * TS - 1) / (2 * TS)), static_cast<unsigned>(a.B));
  const unsigned nt = static_cast<unsigned>(2 * a.D);  // the register cap follows nt
  if (nt > 768)
    ent_reg_kernel<DT, WM, KI, 1024, TS><<<grid, nt, f.total, TESM_LOGGED(st, ent_reg_kernel<DT, WM, KI, 1024, TS>)>>>(a, weff, f);
  else if (nt > 512)
    ent_reg_kernel<DT, WM, KI, 768, TS><<<grid, nt, f.total, TESM_LOGGED(st, ent_reg_kernel<DT, WM, KI, 768, TS>)>>>(a, weff, f);
  else
    ent_reg_kernel<DT, WM, KI, 512, TS><<<grid, nt, f.total, TESM_LOGGED(st, ent_reg_kernel<DT, WM, KI, 512, TS>)>>>(a, weff, f);
}

template <int DT>
static int run_reg(const EntArgs& a, int64_t weff, hipStream_t st) {
  const int wm = weff <= 16 ? 16 : 32;
  const RegLds f = reg_lds(a.D, a.R, weff, wm, DT == kBF16 ? 2 : 4, 2 * kRegTS);
  const int64_t ki = ((2 * kRegTS + weff - 1) * (a.R / 2) + 2 * a.D - 1) / (2 * a.D);  // first-round key items
  if (wm == 16) {
    if (ki <= 2) launch_reg_k<DT, 16, 2>(a, weff, f, st);
    else if (ki == 3) launch_reg_k<DT, 16, 3>(a, weff, f, st);
    else launch_reg_k<DT, 16, 4>(a, weff, f, st);
  } else {
    if (ki <= 2) launch_reg_k<DT, 32, 2>(a, weff, f, st);
    else if (ki == 3) launch_reg_k<DT, 32, 3>(a, weff, f, st);
    else launch_reg_k<DT, 32, 4>(a, weff, f, st);
  }
  return check_launch("entanglement fused (window mix in registers)");
}

// The register-mix form (SISO, quantized outputs): D a multiple of 64 up to 512, an effective window of
// at most 32, LDS within 64 KB.  It runs where neither of the other fused kernels fits (float32 rows of
// 384+ channels, which otherwise take the scores + mix kernels and two activation quantizations: the
// tiny() model's float32 forward 2.92 -> 2.51 ms); where they fit they are faster (configs[3] layer 11.6
// against 14.6 us, the base() preset's own layer 107 against 109 us).  TESM_HIP_NO_ENT_REG=1 (read per
// call) keeps the unfused kernels for those shapes (the tests compare the two bit for bit).
static bool reg_fits(const EntArgs& a, int64_t weff) {
  if (a.mimo || a.H != 1 || a.D % 64 != 0 || a.D > 512 || weff > 32) return false;
  const char* off = std::getenv("TESM_HIP_NO_ENT_REG");
  if (off != nullptr && off[0] == '1') return false;
  return reg_lds(a.D, a.R, weff, weff <= 16 ? 16 : 32, a.dt == kBF16 ? 2 : 4, 2 * kRegTS).total <= 64 * 1024;
}

template <bool QUANT, int KI>
static void launch_fused2(const EntArgs& a, int64_t weff, const Fused2Lds& f2, hipStream_t st) {
  dim3 grid2(static_cast<unsigned>((a.L + kF2TP - 1) / kF2TP), static_cast<unsigned>(a.B));
  if (a.dt == kBF16)
    ent_fused2_kernel<kBF16, QUANT, KI><<<grid2, 512, f2.total, TESM_LOGGED(st, ent_fused2_kernel<kBF16, QUANT, KI>)>>>(a, weff, f2);
  else
    ent_fused2_kernel<kF32, QUANT, KI><<<grid2, 512, f2.total, TESM_LOGGED(st, ent_fused2_kernel<kF32, QUANT, KI>)>>>(a, weff, f2);
}

template <bool QUANT>
static int run_fused2(const EntArgs& a, int64_t weff, hipStream_t st) {
  const Fused2Lds f2 = fused2_lds(a.R, a.D, weff);
  const int64_t rows = kF2TP + weff - 1, half = a.R / 2, nsl = a.D / 8;
  if (rows * nsl <= 512 * 2 && rows * half <= 512 * 2 && kF2TP * half <= 512)
    launch_fused2<QUANT, 2>(a, weff, f2, st);
  else
    launch_fused2<QUANT, 4>(a, weff, f2, st);
  return check_launch("entanglement fused (32 threads per position)");
}

// TESM_HIP_NO_ENT_FUSED2=1 keeps the 16-threads-per-position kernel (a diagnostic switch for
// side-by-side timing and bit-for-bit comparison)
static bool no_f2() {
  static const bool off = [] {
    const char* e = std::getenv("TESM_HIP_NO_ENT_FUSED2");
    return e != nullptr && e[0] == '1';
  }();
  return off;
}

// The 32-threads-per-position form (SISO): D % 16 == 0 up to 512, its load items within 4 / 4 / 2 per
// thread, 16-byte aligned state rows, LDS within 64 KB.
static bool fused2_fits(const EntArgs& a, int64_t weff) {
  if (a.mimo || a.H != 1 || no_f2()) return false;
  const Fused2Lds f2 = fused2_lds(a.R, a.D, weff);
  const int64_t rows = kFusedTP + weff - 1, half = a.R / 2, nsl = a.D / 8;
  return a.D % 16 == 0 && a.D <= 512 && rows * nsl <= 512 * 4 && rows * half <= 512 * 4 && kF2TP * half <= 512 * 2 &&
         weff <= 64 && a.ld_s % 8 == 0 && aligned(a.S, 16) && f2.total <= 64 * 1024;
}

// TESM_HIP_ENT_UNFUSED=1 makes the float-output entry (no int8 codes) take the scores + mix kernels
// instead of the 32-thread fused kernel (read per call: the tests compare the two bit for bit)
static bool ent_unfused_requested() {
  const char* e = std::getenv("TESM_HIP_ENT_UNFUSED");
  return e != nullptr && e[0] == '1';
}

// The 16-threads-per-position form: D up to 512, its LDS within 64 KB.
static bool fused16_fits(const EntArgs& a, int64_t weff) {
  return !a.mimo && a.H == 1 && a.D <= 16 * 16 * kFusedMaxGPT &&
         fused_lds(a.R, a.D, weff, a.dt == kBF16 ? 2 : 4).total <= 64 * 1024;
}

bool ent_fused_ok(const EntArgs& a) {
  if (a.mimo || a.H != 1) return false;
  const int64_t weff = eff_window(a);
  return fused16_fits(a, weff) || reg_fits(a, weff);
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
    const int esz = a.dt == kBF16 ? 2 : 4;
    const FusedLds f = fused_lds(a.R, a.D, weff, esz);
    dim3 grid(static_cast<unsigned>((a.L + kFusedTP - 1) / kFusedTP), static_cast<unsigned>(a.B));
    // the single-issue load path's capacity: 4 key / state items per thread up to window 16 at the
    // base shape, 8 beyond (the kernel falls back to its loops where neither fits)
    const int64_t rows = kFusedTP + weff - 1, half = a.R / 2, nvec = f.dp / (16 / esz);
    auto fits = [&](int64_t si) {
      return rows * half <= 256 * si && kFusedTP * half <= 256 * (si / 2) && rows * nvec <= 256 * si;
    };
    const bool big = !fits(4) && fits(8);
    if (fused2_fits(a, weff)) return run_fused2<true>(a, weff, st);
    if (!fused16_fits(a, weff)) return a.dt == kBF16 ? run_reg<kBF16>(a, weff, st) : run_reg<kF32>(a, weff, st);
    if (a.dt == kBF16) {
      if (big)
        ent_fused_kernel<kBF16, 8><<<grid, 256, f.total, TESM_LOGGED(st, ent_fused_kernel<kBF16, 8>)>>>(a, weff, f);
      else
        ent_fused_kernel<kBF16, 4><<<grid, 256, f.total, TESM_LOGGED(st, ent_fused_kernel<kBF16, 4>)>>>(a, weff, f);
    } else {
      if (big)
        ent_fused_kernel<kF32, 8><<<grid, 256, f.total, TESM_LOGGED(st, ent_fused_kernel<kF32, 8>)>>>(a, weff, f);
      else
        ent_fused_kernel<kF32, 4><<<grid, 256, f.total, TESM_LOGGED(st, ent_fused_kernel<kF32, 4>)>>>(a, weff, f);
    }
    return check_launch("entanglement fused");
  }
  // float outputs only: the same 32-thread kernel without its quantization phase
  if (fused2_fits(a, weff) && !ent_unfused_requested()) return run_fused2<false>(a, weff, st);
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
