// Global causal ternary entanglement for gfx950 (see global.h for the reference mapping).
//
//   score(i, j) = dt(dt(dt(q_i . k_j) / sqrt(H*R)) + bias(rel(i, j)))  for j <= i   (q, k after RoPE)
//   t(i, j)     = +1 / -1 / 0 against +-thr (eval hard threshold), n_i = max(sum_j |t(i, j)|, 1)
//   A_i         = sum_j dt(t(i, j) / dt(n_i)) * S_j
// Both contractions run on the matrix cores with float32 accumulation.  RoPE'd queries and keys are
// computed once (float32 holding dt values).  The scores kernel (one workgroup per causal 64 x 64 tile,
// v_mfma_f32_32x32x16_bf16 for bf16 layers, whose operands are exact in bf16, and
// v_mfma_f32_32x32x2_f32 for float32 ones) writes the decisions as int8 (B, L, ldt) and adds each
// query's nonzero count atomically.  The mix kernel contracts decisions x states: states stored in
// bf16 are read from a (channel, key) transposed copy as bf16 MFMA operands; float32 states (float32
// layers, and MIMO, whose states are float32) feed the f32 MFMA one element per lane, straight from
// the (key, channel) layout.  The four waves of a mix workgroup split the keys of one 32-query x
// 64-channel tile and meet in LDS, and the workgroups run heaviest (latest) query block first.  The
// epilogue is the layer's post-processing (SISO: E = S + scale (A - S), tanh(E), E - S; MIMO: the
// rank merge tanh(A c), (A - S) c).
//
// MFMA 32x32 lane layout used throughout: lane L supplies row L % 32 of A and column L % 32 of B, its
// k values in an order shared by both operands (so any assignment of the contraction index to
// (L / 32, element) that is the same for A and B is a valid product); accumulator element r of lane L
// is D[8 (r / 4) + 4 (L / 32) + r % 4][L % 32].
#include "global.h"

namespace tesm {

namespace {

constexpr int kGB = 64;   // queries / keys per scores tile
constexpr int kMQ = 32;   // queries per mix tile
constexpr int kMC = 64;   // channels per mix tile
constexpr int kMK = 32;   // keys per mix step (one wave's share of the key loop advances by 4 x kMK)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Eight floats holding bf16 values as MFMA operands (truncation is exact for them).
__device__ __forceinline__ bf16x8_t as_bf16x8(const float (&v)[8]) {
  u16x8_t u;
#pragma unroll
  for (int e = 0; e < 8; ++e) u[e] = static_cast<unsigned short>(__float_as_uint(v[e]) >> 16);
  return __builtin_bit_cast(bf16x8_t, u);
}

// Eight int8 decisions in {-1, 0, 1} (two dwords) as bf16 operands: 0x3f80 = 1, 0xbf80 = -1.
__device__ __forceinline__ bf16x8_t tern_bf16x8(uint2 w) {
  u16x8_t u;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t b = ((e < 4 ? w.x : w.y) >> (8 * (e & 3))) & 0xffu;
    u[e] = static_cast<unsigned short>(b ? (0x3f80u | ((b & 0x80u) << 8)) : 0u);
  }
  return __builtin_bit_cast(bf16x8_t, u);
}

__device__ __forceinline__ float tern_f(uint32_t w, int s) {
  return static_cast<float>(static_cast<int8_t>((w >> (8 * s)) & 0xffu));
}

template <int DT>
__global__ __launch_bounds__(256) void global_bias_table_kernel(int64_t n, const float* embed, int64_t P,
                                                                const float* scale, const float* bias, float* table) {
  // eight lanes per entry, each over every eighth frequency; the partial sums meet by shuffles
  const int64_t r = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 3;
  const int part = threadIdx.x & 7;
  const float rel = rnd<DT>(static_cast<float>(r < n ? r : 0));
  constexpr float kPi = 3.14159265358979323846f;
  float ssum = 0.0f, csum = 0.0f;
  for (int64_t p = part; p < P; p += 8) {
    const float fr = rnd<DT>(rnd<DT>(static_cast<float>(p + 1) * kPi) / 1000.0f);
    const float ang = rnd<DT>(rel * fr);
    const float e = embed[p];
    ssum += rnd<DT>(rnd<DT>(sinf(ang)) * e);
    csum += rnd<DT>(rnd<DT>(cosf(ang)) * e);
  }
#pragma unroll
  for (int o = 4; o > 0; o >>= 1) {
    ssum += __shfl_xor(ssum, o);
    csum += __shfl_xor(csum, o);
  }
  if (r >= n || part != 0) return;
  const float b = rnd<DT>(rnd<DT>(ssum) + rnd<DT>(csum));
  table[r] = rnd<DT>(rnd<DT>(b * scale[0]) + bias[0]);
}

// RoPE'd queries (+ cross-layer bias) and keys, once: qr / kr (b, t, c) at [(b*L + t)*RQ + c], RQ = H*R,
// float32 holding dt values, dims of each head in the reference's order.  Also clears the per-query
// decision counts that the scores kernel accumulates.
template <int DT>
__global__ __launch_bounds__(256) void global_rope_kernel(GlobalArgs a, float* qr, float* kr) {
  const int64_t RQ = a.H * a.R, half = a.R / 2;
  const int64_t n = a.B * a.L * a.H * half;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (e < a.B * a.L) a.count[e] = 0;
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

// Load n <= 8 consecutive floats of a RoPE'd row from dim d (zero past RQ).
template <int N>
__device__ __forceinline__ void load_dims(const float* row, int64_t d, int64_t RQ, bool vec, float (&v)[N]) {
  if (vec && d + N <= RQ) {
#pragma unroll
    for (int e = 0; e < N; e += 4) {
      const float4 x = *reinterpret_cast<const float4*>(row + d + e);
      v[e] = x.x;
      v[e + 1] = x.y;
      v[e + 2] = x.z;
      v[e + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = d + e < RQ ? row[d + e] : 0.0f;
  }
}

// One workgroup per causal (64-query block, 64-key block) tile of a batch row, tiles numbered row by
// row of the lower triangle.  Wave w computes keys 32 (w & 1) .. +31 (the A operand) against queries
// 32 (w >> 1) .. +31 (B) over all RoPE'd dims, so each accumulator quad of a lane holds four
// consecutive keys of one query: one dword of decisions per quad.
template <int DT>
__global__ __launch_bounds__(256) void global_scores_kernel(GlobalArgs a, const float* qr, const float* kr,
                                                            int64_t ldt) {
  const int64_t tile = blockIdx.x, b = blockIdx.z;
  int64_t qb = static_cast<int64_t>((sqrtf(8.0f * static_cast<float>(tile) + 1.0f) - 1.0f) * 0.5f);
  while ((qb + 1) * (qb + 2) / 2 <= tile) ++qb;
  while (qb * (qb + 1) / 2 > tile) --qb;
  const int64_t kb = tile - qb * (qb + 1) / 2;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t RQ = a.H * a.R;
  const bool vec = (RQ & 3) == 0;
  const int64_t j0 = kb * kGB + 32 * (w & 1), i0 = qb * kGB + 32 * (w >> 1);
  const int64_t jr = j0 + l32 < a.L ? j0 + l32 : a.L - 1;  // rows past L are computed and discarded
  const int64_t ir = i0 + l32 < a.L ? i0 + l32 : a.L - 1;
  const float* krow = kr + (b * a.L + jr) * RQ;
  const float* qrow = qr + (b * a.L + ir) * RQ;
  f32x16_t acc = {};
  if constexpr (DT == kBF16) {
    for (int64_t d0 = 0; d0 < RQ; d0 += 16) {
      float kv[8], qv[8];
      load_dims<8>(krow, d0 + 8 * h, RQ, vec, kv);
      load_dims<8>(qrow, d0 + 8 * h, RQ, vec, qv);
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(as_bf16x8(kv), as_bf16x8(qv), acc, 0, 0, 0);
    }
  } else {
    for (int64_t d0 = 0; d0 < RQ; d0 += 8) {
      float kv[4], qv[4];
      load_dims<4>(krow, d0 + 4 * h, RQ, vec, kv);
      load_dims<4>(qrow, d0 + 4 * h, RQ, vec, qv);
#pragma unroll
      for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv[s], qv[s], acc, 0, 0, 0);
    }
  }
  const int64_t i = i0 + l32;
  if (i >= a.L) return;
  const float pi = rnd<DT>(static_cast<float>(i));
  int cnt = 0;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const int64_t jb = j0 + 8 * g + 4 * h;
    uint32_t packed = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int64_t j = jb + u;
      int t = 0;
      if (j <= i) {
        const int rel = static_cast<int>(rnd<DT>(pi - rnd<DT>(static_cast<float>(j))));
        const float sv = rnd<DT>(rnd<DT>(rnd<DT>(acc[4 * g + u]) / a.sqrt_div) + a.table[rel]);
        t = sv > a.thr ? 1 : (sv < -a.thr ? -1 : 0);
      }
      cnt += t != 0;
      packed |= static_cast<uint32_t>(static_cast<uint8_t>(static_cast<int8_t>(t))) << (8 * u);
    }
    *reinterpret_cast<uint32_t*>(a.tern + (b * a.L + i) * ldt + jb) = packed;
  }
  cnt += __shfl_xor(cnt, 32);
  if (h == 0 && cnt) atomicAdd(a.count + b * a.L + i, cnt);
}

// bf16 states (b, t, c) -> transposed copy (b, c, key) with pitch ldst, keys L .. ldst-1 zero.  A 64-key x
// 64-channel tile goes through LDS; where the rows allow (16-byte aligned, C % 8 == 0) each thread reads
// 8 channels of one key and writes 8 keys of one channel with single 16-byte accesses.
__global__ __launch_bounds__(256) void global_transpose_kernel(const uint16_t* __restrict__ S, int64_t ld_s,
                                                               int64_t L, int64_t C, uint16_t* __restrict__ s_t,
                                                               int64_t ldst) {
  __shared__ uint16_t t[64][64 + 8];  // [channel][key]; rows of 144 bytes keep 16-byte reads aligned
  const int64_t k0 = static_cast<int64_t>(blockIdx.x) * 64, c0 = static_cast<int64_t>(blockIdx.y) * 64;
  const int64_t b = blockIdx.z;
  const int tid = threadIdx.x;
  const bool vec = (C % 8) == 0 && (ld_s % 8) == 0 && (reinterpret_cast<uintptr_t>(S) % 16) == 0;
  if (vec) {
#pragma unroll
    for (int e = tid; e < 64 * 8; e += 256) {
      const int r = e >> 3, c = 8 * (e & 7);  // r: key, c: first of 8 channels
      const int64_t k = k0 + r, ch = c0 + c;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (k < L && ch < C) v = *reinterpret_cast<const uint4*>(S + (b * L + k) * ld_s + ch);
      const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) t[c + i][r] = static_cast<uint16_t>(w[i >> 1] >> (16 * (i & 1)));
    }
  } else {
    for (int e = tid; e < 64 * 64; e += 256) {
      const int r = e >> 6, c = e & 63;
      const int64_t k = k0 + r, ch = c0 + c;
      t[c][r] = (k < L && ch < C) ? S[(b * L + k) * ld_s + ch] : uint16_t(0);
    }
  }
  __syncthreads();
  // ldst is a multiple of 64 and the copy's base 256-byte aligned: rows of the copy take 16-byte stores
#pragma unroll
  for (int e = tid; e < 64 * 8; e += 256) {
    const int r = e >> 3, k = 8 * (e & 7);  // r: channel, k: first of 8 keys
    const int64_t ch = c0 + r;
    if (ch < C)
      *reinterpret_cast<uint4*>(s_t + (b * C + ch) * ldst + k0 + k) = *reinterpret_cast<const uint4*>(&t[r][k]);
  }
}

template <int DT, int SDT, int NWV>
__device__ __forceinline__ void global_mix_finish(const GlobalArgs& a, const float (&part)[NWV][kMQ][kMC + 4],
                                                  int64_t b, int64_t i, int q, int64_t c0, int cc, int64_t C) {
  if (i >= a.L) return;
  const int n = a.count[b * a.L + i];
  const float winv = rnd<DT>(1.0f / rnd<DT>(static_cast<float>(n > 1 ? n : 1)));  // dt(t / dt(n)) for t = 1
#pragma unroll
  for (int y = 0; y < 8; ++y) {
    const int64_t c = c0 + cc + y;
    if (c >= C) break;
    float A0 = part[0][q][cc + y];
#pragma unroll
    for (int v = 1; v < NWV; ++v) A0 += part[v][q][cc + y];
    const float s = ld<SDT>(a.S, (b * a.L + i) * a.ld_s + c);
    const int64_t o = (b * a.L + i) * a.ld_out + c;
    if (a.mimo) {
      const float A = A0 * winv;
      const float cf = a.coef[c];
      st<DT>(a.e_tanh, o, tanhf_(A * cf));
      st<DT>(a.c_out, o, (A - s) * cf);
    } else {
      const float avg = rnd<DT>(A0 * winv);
      const float e = rnd<DT>(s + rnd<DT>(a.ent_scale * rnd<DT>(avg - s)));
      st<DT>(a.e_tanh, o, tanhf_(e));
      st<DT>(a.c_out, o, e - s);
    }
  }
}

// Decisions x states for one (32-query block, 64-channel block, batch row), the query blocks in
// descending order over the flattened grid.  Wave w takes key steps w, w + 4, ... of kMK keys; the
// partial accumulators meet in LDS and every thread finishes 8 consecutive channels of one query.
// SDT: states dtype; bf16 states come transposed in s_t (pitch ldst).
template <int DT, int SDT, int NWV = 4, int PF = 2>
__global__ __launch_bounds__(NWV * 64) void global_mix_kernel(GlobalArgs a, int64_t ldt, const uint16_t* s_t,
                                                               int64_t ldst, int64_t nqb, int64_t ncb) {
  __shared__ float part[NWV][kMQ][kMC + 4];
  const int64_t flat = blockIdx.x;
  const int64_t b = flat % a.B, cb = (flat / a.B) % ncb, qb = nqb - 1 - flat / (a.B * ncb);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, l32 = lane & 31;
  const int64_t C = a.H * a.D;
  const int64_t i0 = qb * kMQ, c0 = cb * kMC;
  const int64_t kend = a.L < i0 + kMQ ? a.L : i0 + kMQ;  // keys 0 .. kend-1 (decisions past i are 0)
  const int64_t nks = (kend + kMK - 1) / kMK;
  const int64_t ir = i0 + l32 < a.L ? i0 + l32 : a.L - 1;
  const int8_t* trow = a.tern + (b * a.L + ir) * ldt;
  f32x16_t acc0 = {}, acc1 = {};
  if constexpr (SDT == kBF16) {
    const int64_t ca = c0 + l32 < C ? c0 + l32 : C - 1, cbb = c0 + 32 + l32 < C ? c0 + 32 + l32 : C - 1;
    const uint16_t* s0 = s_t + (b * C + ca) * ldst;
    const uint16_t* s1 = s_t + (b * C + cbb) * ldst;
    // PF steps of loads in flight: slot p holds step ks + p * NWV of the current round
    uint2 ta[PF][2];
    uint4 sa[PF][2], sb[PF][2];
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int64_t k = w + p * NWV;
      if (k < nks) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int64_t kk = k * kMK + 16 * u + 8 * h;
          ta[p][u] = *reinterpret_cast<const uint2*>(trow + kk);
          sa[p][u] = *reinterpret_cast<const uint4*>(s0 + kk);
          sb[p][u] = *reinterpret_cast<const uint4*>(s1 + kk);
        }
      }
    }
    for (int64_t ks = w; ks < nks; ks += PF * NWV) {
#pragma unroll
      for (int p = 0; p < PF; ++p) {
        const int64_t k = ks + p * NWV;
        if (k < nks) {
          const uint2 t0 = ta[p][0], t1 = ta[p][1];
          const uint4 a0 = sa[p][0], a1 = sa[p][1], b0 = sb[p][0], b1 = sb[p][1];
          const int64_t kn = k + PF * NWV;
          if (kn < nks) {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int64_t kk = kn * kMK + 16 * u + 8 * h;
              ta[p][u] = *reinterpret_cast<const uint2*>(trow + kk);
              sa[p][u] = *reinterpret_cast<const uint4*>(s0 + kk);
              sb[p][u] = *reinterpret_cast<const uint4*>(s1 + kk);
            }
          }
          const bf16x8_t x0 = tern_bf16x8(t0), x1 = tern_bf16x8(t1);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x0, __builtin_bit_cast(bf16x8_t, a0), acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x0, __builtin_bit_cast(bf16x8_t, b0), acc1, 0, 0, 0);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x1, __builtin_bit_cast(bf16x8_t, a1), acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(x1, __builtin_bit_cast(bf16x8_t, b1), acc1, 0, 0, 0);
        }
      }
    }
  } else {
    // step (g, s) pairs the lanes of half h with key 8 g + 4 h + s: one dword of decisions per g
    const int64_t ca = c0 + l32 < C ? c0 + l32 : C - 1, cbb = c0 + 32 + l32 < C ? c0 + 32 + l32 : C - 1;
    const float* Sf = static_cast<const float*>(a.S);
    for (int64_t ks = w; ks < nks; ks += NWV) {
#pragma unroll
      for (int g = 0; g < kMK / 8; ++g) {
        const int64_t kk = ks * kMK + 8 * g + 4 * h;
        const uint32_t tw = *reinterpret_cast<const uint32_t*>(trow + kk);
        float va[4], vb[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int64_t key = kk + s < a.L ? kk + s : a.L - 1;  // past L the decision is 0
          va[s] = Sf[(b * a.L + key) * a.ld_s + ca];
          vb[s] = Sf[(b * a.L + key) * a.ld_s + cbb];
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const float x = tern_f(tw, s);
          acc0 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, va[s], acc0, 0, 0, 0);
          acc1 = __builtin_amdgcn_mfma_f32_32x32x2f32(x, vb[s], acc1, 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int q = 8 * (r / 4) + 4 * h + (r % 4);
    part[w][q][l32] = acc0[r];
    part[w][q][32 + l32] = acc1[r];
  }
  __syncthreads();
  for (int e = tid; e < kMQ * kMC / 8; e += NWV * 64) {
    const int q = e >> 3, cc = 8 * (e & 7);
    global_mix_finish<DT, SDT, NWV>(a, part, b, i0 + q, q, c0, cc, C);
  }
}

}  // namespace

int launch_global_bias_table(int dt, int64_t n, const float* embed, int64_t P, const float* scale, const float* bias,
                             float* table, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "global bias: dtype must be 0 or 1");
  TESM_REQUIRE(embed && scale && bias && table && P >= 1 && n >= 1, kErrInvalidArg, "global bias: bad arguments");
  const unsigned nb = static_cast<unsigned>((8 * n + 255) / 256);
  if (dt == kBF16)
    global_bias_table_kernel<kBF16><<<nb, 256, 0, TESM_LOGGED(st, global_bias_table_kernel<kBF16>)>>>(n, embed, P, scale, bias, table);
  else
    global_bias_table_kernel<kF32><<<nb, 256, 0, TESM_LOGGED(st, global_bias_table_kernel<kF32>)>>>(n, embed, P, scale, bias, table);
  return check_launch("global bias table");
}

int64_t global_tern_pitch(int64_t L) { return round_up(L, kGB); }

int64_t global_states_t_bytes(int dt, int mimo, int64_t B, int64_t L, int64_t C) {
  return dt == kBF16 && !mimo ? B * C * global_tern_pitch(L) * 2 : 0;
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
  const bool bf16_states = a.dt == kBF16 && !a.mimo;  // SISO states are in the layer dtype, MIMO's float32
  TESM_REQUIRE(!bf16_states || a.states_t, kErrInvalidArg, "global ent: null transposed-states workspace");
  const int64_t C = a.H * a.D;
  const int64_t ldt = global_tern_pitch(a.L);
  const int64_t nqb = (a.L + kGB - 1) / kGB;
  const int64_t ntiles = nqb * (nqb + 1) / 2;
  const int64_t nqm = (a.L + kMQ - 1) / kMQ, ncb = (C + kMC - 1) / kMC;
  TESM_REQUIRE(ntiles <= 0x7fffffff && a.B <= 65535 && nqm * ncb * a.B <= 0x7fffffff, kErrUnsupported,
               "global ent: too large");
  TESM_REQUIRE(2 * a.L < (int64_t(1) << 24), kErrUnsupported, "global ent: sequence too long for the bias table");
  TESM_REQUIRE(a.qr && a.kr, kErrInvalidArg, "global ent: null RoPE workspace");
  const int64_t nrope = std::max(a.B * a.L * a.H * (a.R / 2), a.B * a.L);
  const unsigned nbr = static_cast<unsigned>((nrope + 255) / 256);
  const dim3 gs(static_cast<unsigned>(ntiles), 1, static_cast<unsigned>(a.B));
  const unsigned gm = static_cast<unsigned>(nqm * ncb * a.B);
  if (a.dt == kBF16) {
    global_rope_kernel<kBF16><<<nbr, 256, 0, TESM_LOGGED(st, global_rope_kernel<kBF16>)>>>(a, a.qr, a.kr);
    global_scores_kernel<kBF16><<<gs, 256, 0, TESM_LOGGED(st, global_scores_kernel<kBF16>)>>>(a, a.qr, a.kr, ldt);
    if (a.mimo) {
      global_mix_kernel<kBF16, kF32><<<gm, 256, 0, TESM_LOGGED(st, global_mix_kernel<kBF16, kF32>)>>>(
          a, ldt, nullptr, 0, nqm, ncb);
    } else {
      const dim3 gt(static_cast<unsigned>(ldt / 64), static_cast<unsigned>(ncb), static_cast<unsigned>(a.B));
      global_transpose_kernel<<<gt, 256, 0, TESM_LOGGED(st, global_transpose_kernel)>>>(
          static_cast<const uint16_t*>(a.S), a.ld_s, a.L, C, a.states_t, ldt);
      global_mix_kernel<kBF16, kBF16><<<gm, 256, 0, TESM_LOGGED(st, global_mix_kernel<kBF16, kBF16>)>>>(
          a, ldt, a.states_t, ldt, nqm, ncb);
    }
  } else {
    global_rope_kernel<kF32><<<nbr, 256, 0, TESM_LOGGED(st, global_rope_kernel<kF32>)>>>(a, a.qr, a.kr);
    global_scores_kernel<kF32><<<gs, 256, 0, TESM_LOGGED(st, global_scores_kernel<kF32>)>>>(a, a.qr, a.kr, ldt);
    global_mix_kernel<kF32, kF32><<<gm, 256, 0, TESM_LOGGED(st, global_mix_kernel<kF32, kF32>)>>>(a, ldt, nullptr, 0,
                                                                                                   nqm, ncb);
  }
  return check_launch("global ent");
}

}  // namespace tesm
