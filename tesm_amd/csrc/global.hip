// Global causal ternary entanglement for gfx950 (see global.h for the reference mapping).
//
//   score(i, j) = dt(dt(dt(q_i . k_j) / sqrt(H*R)) + bias(rel(i, j)))  for j <= i   (q, k after RoPE)
//   t(i, j)     = +1 / -1 / 0 against +-thr (eval hard threshold), n_i = max(sum_j |t(i, j)|, 1)
//   A_i         = sum_j dt(t(i, j) / dt(n_i)) * S_j
// RoPE'd queries and keys are computed once; the scores kernel (one workgroup per causal 64 x 64 tile)
// writes the decisions as int8 (B, L, ldt) with per-tile counts,
// the mix kernel streams 64-key tiles of decisions and states through LDS into 4 x 4 register tiles
// and finishes with the layer's post-processing (SISO: E = S + scale (A - S), tanh(E), E - S; MIMO:
// the rank merge tanh(A c), (A - S) c).
#include "global.h"

namespace tesm {

namespace {

constexpr int kGB = 64;  // queries / keys / channels per tile

template <int DT>
__global__ __launch_bounds__(256) void global_bias_table_kernel(int64_t n, const float* embed, int64_t P,
                                                                const float* scale, const float* bias, float* table) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (r >= n) return;
  const float rel = rnd<DT>(static_cast<float>(r));
  constexpr float kPi = 3.14159265358979323846f;
  float ssum = 0.0f, csum = 0.0f;
  for (int64_t p = 0; p < P; ++p) {
    const float fr = rnd<DT>(rnd<DT>(static_cast<float>(p + 1) * kPi) / 1000.0f);
    const float ang = rnd<DT>(rel * fr);
    const float e = embed[p];
    ssum += rnd<DT>(rnd<DT>(sinf(ang)) * e);
    csum += rnd<DT>(rnd<DT>(cosf(ang)) * e);
  }
  const float b = rnd<DT>(rnd<DT>(ssum) + rnd<DT>(csum));
  table[r] = rnd<DT>(rnd<DT>(b * scale[0]) + bias[0]);
}

// RoPE'd queries (+ cross-layer bias) and keys, once: qr / kr (b, t, c) at [(b*L + t)*RQ + c], RQ = H*R,
// float32 holding dt values, dims of each head in the reference's order.
template <int DT>
__global__ __launch_bounds__(256) void global_rope_kernel(GlobalArgs a, float* qr, float* kr) {
  const int64_t RQ = a.H * a.R, half = a.R / 2;
  const int64_t n = a.B * a.L * a.H * half;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e >= n) return;
  const int64_t p = e % half, h = (e / half) % a.H, bt = e / (half * a.H);
  const int64_t t = bt % a.L;
  const float2 cs = a.rope[t * half + p];
  const int64_t qo = bt * a.ld_q + h * a.R, ko = bt * a.ld_k + h * a.R, o = bt * RQ + h * a.R;
  float q1, q2, k1, k2;
  rope_pair<DT>(ld<DT>(a.q, qo + p), ld<DT>(a.q, qo + half + p), cs, q1, q2);
  rope_pair<DT>(ld<DT>(a.k, ko + p), ld<DT>(a.k, ko + half + p), cs, k1, k2);
  if (a.q_add) {
    const int64_t ao = bt * a.ld_qadd + h * a.R;
    q1 = rnd<DT>(q1 + ld<DT>(a.q_add, ao + p));
    q2 = rnd<DT>(q2 + ld<DT>(a.q_add, ao + half + p));
  }
  qr[o + p] = q1;
  qr[o + half + p] = q2;
  kr[o + p] = k1;
  kr[o + half + p] = k2;
}

// One workgroup per causal (64-query block, 64-key block) tile of a batch row; thread
// (tid / 16, tid % 16) owns queries 4*(tid/16) .. +3 and keys 4*(tid%16) .. +3.  The RoPE'd dims are
// staged 64 at a time; the dot products run over them in order.  Writes the tile's decisions and
// its per-query nonzero counts (part[(b*L + i)*nkb + kb]).
template <int DT>
__global__ __launch_bounds__(256) void global_scores_kernel(GlobalArgs a, const float* qr, const float* kr,
                                                            int64_t ldt, int32_t* part, int64_t nkb) {
  __shared__ float qs[64][kGB + 4];  // [dim in chunk][query]
  __shared__ float ks[64][kGB + 4];  // [dim in chunk][key]
  const int64_t kb = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
  if (kb > qb) return;
  const int tid = threadIdx.x;
  const int tq = 4 * (tid >> 4), tk = 4 * (tid & 15);
  const int64_t i0 = qb * kGB, j0 = kb * kGB;
  const int64_t RQ = a.H * a.R;
  float dot[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) dot[x][y] = 0.0f;
  for (int64_t d0 = 0; d0 < RQ; d0 += 64) {
    const int nd = static_cast<int>(RQ - d0 < 64 ? RQ - d0 : 64);
    __syncthreads();
    for (int e = tid; e < 64 * 64; e += 256) {
      const int row = e >> 6, d = e & 63;
      const int64_t ti = i0 + row, tj = j0 + row;
      if (d < nd) {
        qs[d][row] = ti < a.L ? qr[(b * a.L + ti) * RQ + d0 + d] : 0.0f;
        ks[d][row] = tj < a.L ? kr[(b * a.L + tj) * RQ + d0 + d] : 0.0f;
      }
    }
    __syncthreads();
    for (int d = 0; d < nd; ++d) {
      const float4 qv = *reinterpret_cast<const float4*>(&qs[d][tq]);
      const float4 kv = *reinterpret_cast<const float4*>(&ks[d][tk]);
      const float q4[4] = {qv.x, qv.y, qv.z, qv.w}, k4[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) dot[x][y] += q4[x] * k4[y];
    }
  }
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int64_t i = i0 + tq + x;
    int cnt = 0;
    uint32_t packed = 0;
    if (i < a.L) {
      const float pi = rnd<DT>(static_cast<float>(i));
#pragma unroll
      for (int y = 0; y < 4; ++y) {
        const int64_t j = j0 + tk + y;
        int t = 0;
        if (j <= i) {
          const int rel = static_cast<int>(rnd<DT>(pi - rnd<DT>(static_cast<float>(j))));
          const float sv = rnd<DT>(rnd<DT>(rnd<DT>(dot[x][y]) / a.sqrt_div) + a.table[rel]);
          t = sv > a.thr ? 1 : (sv < -a.thr ? -1 : 0);
        }
        cnt += t != 0;
        packed |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(t))) << (8 * y);
      }
      *reinterpret_cast<uint32_t*>(a.tern + (b * a.L + i) * ldt + j0 + tk) = packed;
    }
    // the 16 lanes holding one query row are consecutive lanes of a wave
    for (int o = 8; o > 0; o >>= 1) cnt += __shfl_xor(cnt, o);
    if ((tid & 15) == 0 && i < a.L) part[(b * a.L + i) * nkb + kb] = cnt;
  }
}

// One workgroup per (64-channel block, 64-query block, batch row); thread (tid / 16, tid % 16) owns
// queries 4*(tid/16) .. +3 and channels 4*(tid%16) .. +3.  SDT: states dtype.
template <int DT, int SDT>
__global__ __launch_bounds__(256) void global_mix_kernel(GlobalArgs a, int64_t ldt, int64_t nqb_all) {
  __shared__ float ts[kGB][kGB + 4];  // [key][query] decisions as floats
  __shared__ float ss[kGB][kGB + 4];  // [key][channel] states
  const int64_t cb = blockIdx.x, qb = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int tq = 4 * (tid >> 4), tc = 4 * (tid & 15);
  const int64_t i0 = qb * kGB, c0 = cb * kGB;
  const int64_t C = a.H * a.D;
  float acc[4][4];
#pragma unroll
  for (int x = 0; x < 4; ++x)
#pragma unroll
    for (int y = 0; y < 4; ++y) acc[x][y] = 0.0f;
  for (int64_t kb = 0; kb <= qb; ++kb) {
    const int64_t j0 = kb * kGB;
    __syncthreads();
    for (int e = tid; e < kGB * kGB; e += 256) {
      const int r = e >> 6, c = e & 63;  // r: query (decisions) / key (states)
      const int64_t i = i0 + r, j = j0 + r;
      ts[c][r] = i < a.L ? static_cast<float>(a.tern[(b * a.L + i) * ldt + j0 + c]) : 0.0f;
      ss[r][c] = (j < a.L && c0 + c < C) ? ld<SDT>(a.S, (b * a.L + j) * a.ld_s + c0 + c) : 0.0f;
    }
    __syncthreads();
    const int64_t jn = (a.L - j0 < kGB) ? a.L - j0 : kGB;
    for (int j = 0; j < jn; ++j) {
      const float4 tv = *reinterpret_cast<const float4*>(&ts[j][tq]);
      const float4 sv = *reinterpret_cast<const float4*>(&ss[j][tc]);
      const float tq4[4] = {tv.x, tv.y, tv.z, tv.w}, sc4[4] = {sv.x, sv.y, sv.z, sv.w};
#pragma unroll
      for (int x = 0; x < 4; ++x)
#pragma unroll
        for (int y = 0; y < 4; ++y) acc[x][y] = __builtin_fmaf(tq4[x], sc4[y], acc[x][y]);
    }
  }
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int64_t i = i0 + tq + x;
    if (i >= a.L) continue;
    int n = 0;
    for (int64_t kb = 0; kb <= qb; ++kb) n += a.count[(b * a.L + i) * nqb_all + kb];
    const float winv = rnd<DT>(1.0f / rnd<DT>(static_cast<float>(n > 1 ? n : 1)));  // dt(t / dt(n)) for t = 1
#pragma unroll
    for (int y = 0; y < 4; ++y) {
      const int64_t c = c0 + tc + y;
      if (c >= C) continue;
      const float s = ld<SDT>(a.S, (b * a.L + i) * a.ld_s + c);
      const int64_t o = (b * a.L + i) * a.ld_out + c;
      if (a.mimo) {
        const float A = acc[x][y] * winv;
        const float cf = a.coef[c];
        st<DT>(a.e_tanh, o, tanhf_(A * cf));
        st<DT>(a.c_out, o, (A - s) * cf);
      } else {
        const float avg = rnd<DT>(acc[x][y] * winv);
        const float e = rnd<DT>(s + rnd<DT>(a.ent_scale * rnd<DT>(avg - s)));
        st<DT>(a.e_tanh, o, tanhf_(e));
        st<DT>(a.c_out, o, e - s);
      }
    }
  }
}

}  // namespace

int launch_global_bias_table(int dt, int64_t n, const float* embed, int64_t P, const float* scale, const float* bias,
                             float* table, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "global bias: dtype must be 0 or 1");
  TESM_REQUIRE(embed && scale && bias && table && P >= 1 && n >= 1, kErrInvalidArg, "global bias: bad arguments");
  const unsigned nb = static_cast<unsigned>((n + 255) / 256);
  if (dt == kBF16)
    global_bias_table_kernel<kBF16><<<nb, 256, 0, TESM_LOGGED(st, global_bias_table_kernel<kBF16>)>>>(n, embed, P, scale, bias, table);
  else
    global_bias_table_kernel<kF32><<<nb, 256, 0, TESM_LOGGED(st, global_bias_table_kernel<kF32>)>>>(n, embed, P, scale, bias, table);
  return check_launch("global bias table");
}

int64_t global_tern_pitch(int64_t L) { return round_up(L, kGB); }

int64_t global_ws_bytes(int64_t B, int64_t L, int64_t RQ) {
  const int64_t nkb = (L + kGB - 1) / kGB;
  return round_up(B * L * global_tern_pitch(L), 256) + round_up(B * L * nkb * 4, 256) + round_up(2 * L * 4, 256) +
         2 * round_up(B * L * RQ * 4, 256);
}

int launch_global_ent(const GlobalArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "global ent: dtype must be 0 or 1");
  TESM_REQUIRE(a.B >= 0 && a.L >= 0 && a.H >= 1 && a.R >= 2 && a.R % 2 == 0 && a.D >= 1, kErrInvalidArg,
               "global ent: bad sizes (need an even ent_rank)");
  if (a.B == 0 || a.L == 0) return kOk;
  TESM_REQUIRE(a.q && a.k && a.rope && a.table && a.S && a.e_tanh && a.c_out && a.tern && a.count, kErrInvalidArg,
               "global ent: null pointer");
  TESM_REQUIRE(!a.mimo || a.coef, kErrInvalidArg, "global ent: MIMO needs the merge factors");
  TESM_REQUIRE(!a.mimo || !a.q_add, kErrInvalidArg, "global ent: MIMO has no cross-layer query");
  const int64_t ldt = global_tern_pitch(a.L);
  const int64_t nqb = (a.L + kGB - 1) / kGB;
  const int64_t ncb = (a.H * a.D + kGB - 1) / kGB;
  TESM_REQUIRE(nqb <= 65535 && a.B <= 65535 && ncb <= 0x7fffffff, kErrUnsupported, "global ent: too large");
  TESM_REQUIRE(2 * a.L < (int64_t(1) << 24), kErrUnsupported, "global ent: sequence too long for the bias table");
  TESM_REQUIRE(a.qr && a.kr, kErrInvalidArg, "global ent: null RoPE workspace");
  const int64_t nrope = a.B * a.L * a.H * (a.R / 2);
  const unsigned nbr = static_cast<unsigned>((nrope + 255) / 256);
  const dim3 gs(static_cast<unsigned>(nqb), static_cast<unsigned>(nqb), static_cast<unsigned>(a.B));
  const dim3 gm(static_cast<unsigned>(ncb), static_cast<unsigned>(nqb), static_cast<unsigned>(a.B));
  if (a.dt == kBF16) {
    global_rope_kernel<kBF16><<<nbr, 256, 0, TESM_LOGGED(st, global_rope_kernel<kBF16>)>>>(a, a.qr, a.kr);
    global_scores_kernel<kBF16><<<gs, 256, 0, TESM_LOGGED(st, global_scores_kernel<kBF16>)>>>(a, a.qr, a.kr, ldt, a.count, nqb);
    if (a.mimo)
      global_mix_kernel<kBF16, kF32><<<gm, 256, 0, TESM_LOGGED(st, global_mix_kernel<kBF16, kF32>)>>>(a, ldt, nqb);
    else
      global_mix_kernel<kBF16, kBF16><<<gm, 256, 0, TESM_LOGGED(st, global_mix_kernel<kBF16, kBF16>)>>>(a, ldt, nqb);
  } else {
    global_rope_kernel<kF32><<<nbr, 256, 0, TESM_LOGGED(st, global_rope_kernel<kF32>)>>>(a, a.qr, a.kr);
    global_scores_kernel<kF32><<<gs, 256, 0, TESM_LOGGED(st, global_scores_kernel<kF32>)>>>(a, a.qr, a.kr, ldt, a.count, nqb);
    global_mix_kernel<kF32, kF32><<<gm, 256, 0, TESM_LOGGED(st, global_mix_kernel<kF32, kF32>)>>>(a, ldt, nqb);
  }
  return check_launch("global ent");
}

}  // namespace tesm
