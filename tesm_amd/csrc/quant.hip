// BitLinear quantization kernels for gfx950:
//   * per-token int8 activation codes      (reference tesm_ssm/modules/tesm.py:206-209)
//   * per-tensor absmean ternary scale      (tesm.py:211-212)
//   * ternary codes packed 4 per byte       (tesm.py:213-214 + tesm_ssm/utils/int2_quantization.py:21-58)
//   * unpacking back to signed codes        (int2_quantization.py:68-93)
//
// Code buffers feed the INT2 x INT8 GEMV/GEMM, which unpacks a packed dword
// W (16 codes, code k = 4j + s of the group in bits 8j+2s) as the four dwords
// (W >> 2s) & 0x03030303.  Byte j of dword s then holds code 4j + s, so the
// activation codes are written in the matching order ("layout 1"): within each
// group of 16, byte 4s + j holds x[4j + s].  Layout 0 is plain row-major.
#include "tesm_hip_internal.h"

namespace tesm {


// LPR lanes per row (64 / LPR rows per wave, 4 waves per workgroup).  Each lane owns code groups
// lane, lane + LPR, ... ; with G > 0 its G groups stay in registers between the amax and the code
// pass (loaded in straight-line code, all in flight together, for 16-byte aligned rows with
// K % 16 == 0), with G == 0 (very wide rows) the row is read twice.
template <int DT, bool VEC, int LPR, int G>
__global__ __launch_bounds__(256) void quant_act_kernel(const void* __restrict__ x, int64_t M, int64_t K,
                                                        int64_t ldx, float eps, int layout, int8_t* __restrict__ q,
                                                        int64_t ldq, float* __restrict__ s_out,
                                                        int32_t* __restrict__ rowsum, int* __restrict__ zero_p,
                                                        int64_t zero_n, QuantSet second) {
  constexpr int RPW = 64 / LPR;
  if (blockIdx.y == 0) {
    // side job for a later kernel of the same stream: clear zero_n ints (a fill launch saved)
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < zero_n;
         i += static_cast<int64_t>(gridDim.x) * 256)
      zero_p[i] = 0;
  } else {  // the second matrix of a two-matrix launch: same shape, its own codes, scales and sums
    x = second.x;
    q = second.q;
    s_out = second.s;
    rowsum = second.rs;
  }
  const int lane = threadIdx.x & 63;
  const int g0 = lane & (LPR - 1);
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * RPW + lane / LPR;
  if (row >= M) return;  // whole lane groups leave together
  const int64_t base = row * ldx;
  const int64_t ngroups = ldq / 16;

  float amax = 0.0f;
  int32_t rs = 0;
  if constexpr (G > 0) {
    float v[G][16];
    if (VEC && K % 16 == 0) {  // straight-line loads, all in flight together
      load_groups<DT, G, LPR>(x, base, K, g0, v);
    } else {
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        const int64_t g = g0 + LPR * gi;
        if (g < ngroups) {
          load_group<DT, VEC>(x, base, K, g, v[gi]);
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) v[gi][i] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi)
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[gi][i]));
    amax = wave_max<LPR>(amax);
    const float sc = act_scale<DT>(amax, eps);
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int64_t g = g0 + LPR * gi;
      if (g < ngroups) *reinterpret_cast<uint4*>(q + row * ldq + 16 * g) = group_codes<DT>(v[gi], sc, layout, rs);
    }
    if (g0 == 0) s_out[row] = sc;
  } else {
    for (int64_t g = g0; g < ngroups; g += LPR) {
      float v[16];
      load_group<DT, VEC>(x, base, K, g, v);
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
    }
    amax = wave_max<LPR>(amax);
    const float sc = act_scale<DT>(amax, eps);
    for (int64_t g = g0; g < ngroups; g += LPR) {
      float v[16];
      load_group<DT, VEC>(x, base, K, g, v);
      *reinterpret_cast<uint4*>(q + row * ldq + 16 * g) = group_codes<DT>(v, sc, layout, rs);
    }
    if (g0 == 0) s_out[row] = sc;
  }
  rs = wave_sum_i<LPR>(rs);
  if (g0 == 0 && rowsum) rowsum[row] = rs;
}

template <int DT, bool VEC, int LPR, int G>
void run_quant(const void* x, int64_t M, int64_t K, int64_t ldx, float eps, int layout, int8_t* q, int64_t ldq,
               float* s_x, int32_t* rowsum, int* zero_p, int64_t zero_n, const QuantSet& q2, hipStream_t st) {
  constexpr int RPB = 4 * (64 / LPR);
  const unsigned nb = static_cast<unsigned>(std::max<int64_t>((M + RPB - 1) / RPB, zero_n > 0 ? 1 : 0));
  const dim3 grid(nb, q2.x ? 2u : 1u);
  quant_act_kernel<DT, VEC, LPR, G><<<grid, 256, 0, TESM_LOGGED(st, quant_act_kernel<DT, VEC, LPR, G>)>>>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zero_p, zero_n, q2);
}

template <int DT, bool VEC>
void dispatch_quant(const void* x, int64_t M, int64_t K, int64_t ldx, float eps, int layout, int8_t* q, int64_t ldq,
                    float* s_x, int32_t* rowsum, int* zp, int64_t zn, const QuantSet& q2, hipStream_t st) {
  const int64_t ng = ldq / 16;
  // many rows of 24-64 groups (K 384-1024): 16 lanes per row with 2-4 groups each, so that an 8192-row
  // batch runs two waves per SIMD (measured at M 8192, K 768 on one box: 6.2 us against 6.8 us for 8 lanes
  // per row with 6 groups each, which in turn had taken 5.2 against 6.4 us for 64 lanes per row); short
  // batches keep more lanes per row
  if (M >= 2048 && ng > 16 && ng <= 64) {
    switch ((ng + 15) / 16) {
      case 2: return run_quant<DT, VEC, 16, 2>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
      case 3: return run_quant<DT, VEC, 16, 3>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
      default: return run_quant<DT, VEC, 16, 4>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
    }
  }
  if (ng <= 4) return run_quant<DT, VEC, 4, 1>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 8) return run_quant<DT, VEC, 8, 1>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 16) return run_quant<DT, VEC, 16, 1>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 32) return run_quant<DT, VEC, 32, 1>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 64) return run_quant<DT, VEC, 64, 1>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 128) return run_quant<DT, VEC, 64, 2>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 256) return run_quant<DT, VEC, 64, 4>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  if (ng <= 512) return run_quant<DT, VEC, 64, 8>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
  return run_quant<DT, VEC, 64, 0>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zp, zn, q2, st);
}

static int quant_act_impl(const void* x, int dt, int64_t M, int64_t K, int64_t ldx, float eps, int layout, int8_t* q,
                          int64_t ldq, float* s_x, int32_t* rowsum, hipStream_t st, int* zero_p, int64_t zero_n,
                          const QuantSet& q2) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "quant_act: dtype must be 0 (f32) or 1 (bf16)");
  TESM_REQUIRE(M >= 0 && K >= 1 && ldx >= K, kErrInvalidArg, "quant_act: need M >= 0, K >= 1, ldx >= K");
  TESM_REQUIRE(ldq >= K && ldq % 16 == 0, kErrInvalidArg, "quant_act: ldq must be >= K and a multiple of 16");
  TESM_REQUIRE(layout == 0 || layout == 1, kErrInvalidArg, "quant_act: layout must be 0 or 1");
  TESM_REQUIRE(M == 0 || (x && q && s_x), kErrInvalidArg, "quant_act: null pointer");
  TESM_REQUIRE(aligned(q, 16), kErrAlignment, "quant_act: code buffer must be 16-byte aligned");
  TESM_REQUIRE(zero_n == 0 || zero_p, kErrInvalidArg, "quant_act: null range to clear");
  TESM_REQUIRE(!q2.x || M == 0 || (q2.q && q2.s && aligned(q2.q, 16)), kErrInvalidArg,
               "quant_act: the second matrix needs 16-byte aligned codes and a scale buffer");
  if (M == 0 && zero_n == 0) return kOk;  // with M == 0 one workgroup still clears the side range
  const int esz = dt == kBF16 ? 2 : 4;
  const bool vec = aligned(x, 16) && (!q2.x || aligned(q2.x, 16)) && (ldx * esz) % 16 == 0;
  if (dt == kBF16) {
    if (vec) dispatch_quant<kBF16, true>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zero_p, zero_n, q2, st);
    else dispatch_quant<kBF16, false>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zero_p, zero_n, q2, st);
  } else {
    if (vec) dispatch_quant<kF32, true>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zero_p, zero_n, q2, st);
    else dispatch_quant<kF32, false>(x, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, zero_p, zero_n, q2, st);
  }
  return check_launch("quant_act");
}

int launch_quant_act(const void* x, int dt, int64_t M, int64_t K, int64_t ldx, float eps, int layout, int8_t* q,
                     int64_t ldq, float* s_x, int32_t* rowsum, hipStream_t st, int* zero_p, int64_t zero_n) {
  return quant_act_impl(x, dt, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, st, zero_p, zero_n, QuantSet{});
}

int launch_quant_act2(const void* x0, const void* x1, int dt, int64_t M, int64_t K, int64_t ldx, float eps,
                      int8_t* q0, int8_t* q1, int64_t ldq, float* s0, float* s1, int32_t* rs0, int32_t* rs1,
                      hipStream_t st) {
  TESM_REQUIRE(x1 != nullptr, kErrInvalidArg, "quant_act: null second matrix");
  QuantSet q2;
  q2.x = x1;
  q2.q = q1;
  q2.s = s1;
  q2.rs = rs1;
  return quant_act_impl(x0, dt, M, K, ldx, eps, 1, q0, ldq, s0, rs0, st, nullptr, 0, q2);
}

// ---------------------------------------------------------------------------
// absmean weight scale: s_w = 1 / max(mean|w|, eps), c_w = 1 / s_w (the value of a
// dequantized +1 code).  Deterministic: fixed grid, fixed reduction order, fp64 sums.
// ---------------------------------------------------------------------------
constexpr int kAbsmeanBlocks = 512;

template <int DT>
__global__ __launch_bounds__(256) void absmean_partial_kernel(const void* __restrict__ w, int64_t n,
                                                              double* __restrict__ partial) {
  __shared__ double red[4];
  double acc = 0.0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
    acc += fabs(static_cast<double>(ld<DT>(w, i)));
  acc = wave_sum_d(acc);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) partial[blockIdx.x] = (red[0] + red[1]) + (red[2] + red[3]);
}

template <int DT>
__global__ __launch_bounds__(64) void absmean_final_kernel(const double* __restrict__ partial, int np, int64_t n,
                                                           float eps, float* __restrict__ s_w,
                                                           float* __restrict__ c_w) {
  double acc = 0.0;
  for (int i = threadIdx.x; i < np; i += 64) acc += partial[i];
  acc = wave_sum_d(acc);
  if (threadIdx.x == 0) {
    float m = rnd<DT>(static_cast<float>(acc / static_cast<double>(n)));
    const float e = rnd<DT>(eps);
    m = m < e ? e : m;
    const float s = rnd<DT>(1.0f / m);
    s_w[0] = s;
    c_w[0] = rnd<DT>(1.0f / s);
  }
}

int launch_absmean(const void* w, int dt, int64_t n, float eps, double* ws, float* s_w, float* c_w, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "absmean: dtype must be 0 (f32) or 1 (bf16)");
  TESM_REQUIRE(n >= 1 && w && ws && s_w && c_w, kErrInvalidArg, "absmean: need n >= 1 and non-null pointers");
  const int nb = static_cast<int>(std::min<int64_t>(kAbsmeanBlocks, (n + 255) / 256));
  if (dt == kBF16) {
    absmean_partial_kernel<kBF16><<<nb, 256, 0, TESM_LOGGED(st, absmean_partial_kernel<kBF16>)>>>(w, n, ws);
    absmean_final_kernel<kBF16><<<1, 64, 0, TESM_LOGGED(st, absmean_final_kernel<kBF16>)>>>(ws, nb, n, eps, s_w, c_w);
  } else {
    absmean_partial_kernel<kF32><<<nb, 256, 0, TESM_LOGGED(st, absmean_partial_kernel<kF32>)>>>(w, n, ws);
    absmean_final_kernel<kF32><<<1, 64, 0, TESM_LOGGED(st, absmean_final_kernel<kF32>)>>>(ws, nb, n, eps, s_w, c_w);
  }
  return check_launch("absmean");
}

// ---------------------------------------------------------------------------
// INT2 packing: code = clamp(rne(w * s_w), -1, 1) + 1, four codes per byte, code of
// k = 4j + i in bits 2i..2i+1 of byte j, bytes past ceil(K/4) and codes past K hold
// code 1 (value 0).  One thread per packed byte.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void pack_kernel(const void* __restrict__ w, int64_t N, int64_t K, int64_t ldw,
                                                   const float* __restrict__ s_w, int per_row,
                                                   uint8_t* __restrict__ packed, int64_t ldp) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= N * ldp) return;
  const int64_t n = idx / ldp, j = idx - n * ldp;
  const float s = per_row ? s_w[n] : s_w[0];
  uint32_t byte = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t k = 4 * j + i;
    uint32_t u = 1;
    if (k < K) {
      float r = rintf(rnd<DT>(ld<DT>(w, n * ldw + k) * s));
      r = fminf(fmaxf(r, -1.0f), 1.0f);
      u = static_cast<uint32_t>(static_cast<int>(r) + 1);
    }
    byte |= u << (2 * i);
  }
  packed[idx] = static_cast<uint8_t>(byte);
}

int launch_pack(const void* w, int dt, int64_t N, int64_t K, int64_t ldw, const float* s_w, int per_row,
                uint8_t* packed, int64_t ldp, hipStream_t st) {
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "pack_w_i2: dtype must be 0 (f32) or 1 (bf16)");
  TESM_REQUIRE(N >= 0 && K >= 1 && ldw >= K && ldp >= (K + 3) / 4, kErrInvalidArg,
               "pack_w_i2: need K >= 1, ldw >= K, ldp >= ceil(K/4)");
  TESM_REQUIRE(N == 0 || (w && s_w && packed), kErrInvalidArg, "pack_w_i2: null pointer");
  if (N == 0) return kOk;
  const int64_t total = N * ldp;
  const unsigned nb = static_cast<unsigned>((total + 255) / 256);
  if (dt == kBF16)
    pack_kernel<kBF16><<<nb, 256, 0, TESM_LOGGED(st, pack_kernel<kBF16>)>>>(w, N, K, ldw, s_w, per_row, packed, ldp);
  else
    pack_kernel<kF32><<<nb, 256, 0, TESM_LOGGED(st, pack_kernel<kF32>)>>>(w, N, K, ldw, s_w, per_row, packed, ldp);
  return check_launch("pack_w_i2");
}

__global__ __launch_bounds__(256) void unpack_kernel(const uint8_t* __restrict__ packed, int64_t N, int64_t K,
                                                     int64_t ldp, int8_t* __restrict__ codes, int64_t ldc) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= N * K) return;
  const int64_t n = idx / K, k = idx - n * K;
  const int u = (packed[n * ldp + k / 4] >> (2 * (k & 3))) & 3;
  codes[n * ldc + k] = static_cast<int8_t>(u - 1);
}

int launch_unpack(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* codes, int64_t ldc,
                  hipStream_t st) {
  TESM_REQUIRE(N >= 0 && K >= 1 && ldp >= (K + 3) / 4 && ldc >= K, kErrInvalidArg,
               "unpack_w_i2: need K >= 1, ldp >= ceil(K/4), ldc >= K");
  TESM_REQUIRE(N == 0 || (packed && codes), kErrInvalidArg, "unpack_w_i2: null pointer");
  if (N == 0) return kOk;
  const unsigned nb = static_cast<unsigned>((N * K + 255) / 256);
  unpack_kernel<<<nb, 256, 0, TESM_LOGGED(st, unpack_kernel)>>>(packed, N, K, ldp, codes, ldc);
  return check_launch("unpack_w_i2");
}

}  // namespace tesm
