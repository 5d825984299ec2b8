// Residual add + RMSNorm of the TESM block, with optional per-token int8 codes of the result.
//
// Reference semantics (tesm_ssm/modules/block.py):
//   residual = hidden + residual            (block.py:28; the add in the promoted dtype)
//   h = norm(residual.to(dtype))             (block.py:29)
//   residual = residual.to(float32)          (block.py:30-31, residual_in_fp32)
//   RMSNorm: x * rsqrt(mean(x^2) + eps) * w  (block.py:13-16), every op rounded to the module dtype
// The codes are the next BitLinear's per-token activation quantization (tesm.py:206-209) of h, in
// the product layout ("layout 1"), so the normalised row need not be written when only a BitLinear
// reads it (the feed-forward after norm2).
//
// One workgroup of 256 threads per row; the row's normalised inputs are kept in LDS between the
// passes (D <= 16384).
#include "norm.h"

namespace tesm {

namespace {

constexpr int kNormThreads = 256;

template <int DT>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(NormArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_norm[];
  float* xin = lds_norm;          // D  residual.to(dtype)
  float* red = lds_norm + a.D;    // 8  block reductions
  int* redi = reinterpret_cast<int*>(red + 4);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m = blockIdx.x;
  const int D = static_cast<int>(a.D);
  const void* xr = static_cast<const char*>(a.x) + m * a.ld_x * (DT == kBF16 ? 2 : 4);

  // 1. residual add, residual out, x.pow(2) summed in float
  float ss = 0.0f;
  for (int j = tid; j < D; j += kNormThreads) {
    float s = ld<DT>(xr, j);
    if (a.res) {
      const float r = a.res_dt == kBF16 ? ld<kBF16>(a.res, m * a.ld_res + j) : ld<kF32>(a.res, m * a.ld_res + j);
      // hidden + residual in the promoted dtype: float32 if either operand is, else the module dtype
      s = (a.res_dt == kF32 || DT == kF32) ? s + r : rnd<DT>(s + r);
    }
    if (a.res_out) {
      if (a.res_out_dt == kBF16)
        st<kBF16>(a.res_out, m * a.ld_res_out + j, s);
      else
        st<kF32>(a.res_out, m * a.ld_res_out + j, s);
    }
    const float x = rnd<DT>(s);
    xin[j] = x;
    ss += rnd<DT>(x * x);
  }
  ss = wave_sum_f<64>(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  // 2. mean, + eps, rsqrt (each rounded to the module dtype)
  const float var = rnd<DT>(ss / static_cast<float>(D));
  const float rs = rnd<DT>(1.0f / sqrtf(rnd<DT>(var + a.eps)));
  // 3. y = x * rsqrt(..) * weight
  float amax = 0.0f;
  for (int j = tid; j < D; j += kNormThreads) {
    const float y = rnd<DT>(rnd<DT>(xin[j] * rs) * ld<DT>(a.weight, j));
    if (a.y) st<DT>(a.y, m * a.ld_y + j, y);
    xin[j] = y;
    amax = fmaxf(amax, fabsf(y));
  }
  if (!a.q) return;
  // 4. per-token int8 codes of y (layout 1)
  amax = wave_max<64>(amax);
  __syncthreads();  // every wave is done reading red[] above
  if (lane == 0) red[wave] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = act_scale<DT>(amax, a.bit_eps);
  int8_t* qrow = a.q + m * a.ldq;
  int sum = 0;
  for (int j = tid; j < D; j += kNormThreads) {
    const int c = act_code<DT>(xin[j], sc);
    sum += c;
    qrow[(j & ~15) + layout1_pos(j & 15)] = static_cast<int8_t>(c);
  }
  for (int64_t j = D + tid; j < a.ldq; j += kNormThreads)  // padding codes: 0
    qrow[(j & ~static_cast<int64_t>(15)) + layout1_pos(static_cast<int>(j & 15))] = 0;
  sum = wave_sum_i<64>(sum);
  if (lane == 0) redi[wave] = sum;
  __syncthreads();
  if (tid == 0) {
    a.s_x[m] = sc;
    a.rowsum[m] = (redi[0] + redi[1]) + (redi[2] + redi[3]);
  }
}

}  // namespace

int launch_add_rmsnorm(const NormArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "rmsnorm: dtype must be 0 or 1");
  TESM_REQUIRE(a.M >= 0 && a.D >= 1 && a.D <= kNormMaxD, kErrUnsupported, "rmsnorm: need 1 <= D <= 16384");
  TESM_REQUIRE(a.x && a.weight && a.ld_x >= a.D, kErrInvalidArg, "rmsnorm: need x (ld_x >= D) and weight");
  TESM_REQUIRE(!a.res || ((a.res_dt == kF32 || a.res_dt == kBF16) && a.ld_res >= a.D), kErrInvalidArg,
               "rmsnorm: bad residual operand");
  TESM_REQUIRE(!a.res_out || ((a.res_out_dt == kF32 || a.res_out_dt == kBF16) && a.ld_res_out >= a.D),
               kErrInvalidArg, "rmsnorm: bad residual output");
  TESM_REQUIRE(!a.y || a.ld_y >= a.D, kErrInvalidArg, "rmsnorm: ld_y < D");
  TESM_REQUIRE(!a.q || (a.s_x && a.rowsum && a.ldq >= kpad(a.D) && a.ldq % 16 == 0), kErrInvalidArg,
               "rmsnorm: codes need s_x, rowsum and ldq >= kpad(D), a multiple of 16");
  TESM_REQUIRE(a.y || a.q || a.res_out, kErrInvalidArg, "rmsnorm: nothing to write");
  if (a.M == 0) return kOk;
  const size_t lds = static_cast<size_t>(a.D + 8) * sizeof(float);
  const dim3 grid(static_cast<unsigned>(a.M));
  if (a.dt == kBF16)
    add_rmsnorm_kernel<kBF16><<<grid, kNormThreads, lds, TESM_LOGGED(st, add_rmsnorm_kernel<kBF16>)>>>(a);
  else
    add_rmsnorm_kernel<kF32><<<grid, kNormThreads, lds, TESM_LOGGED(st, add_rmsnorm_kernel<kF32>)>>>(a);
  return check_launch("rmsnorm");
}

}  // namespace tesm
