// Shared device/host helpers for the TESM gfx950 kernels.
//
// Element types at the C-ABI are tagged by an int: 0 = float32, 1 = bfloat16
// (raw 16-bit patterns, round-to-nearest-even on every store).  Every float
// operation that the reference's torch path rounds to the module dtype is
// rounded here at the same point (`rnd<DT>`), so that bf16 results follow the
// reference op by op.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

namespace tesm {

enum Dtype : int { kF32 = 0, kBF16 = 1 };

// ---------------------------------------------------------------------------
// bf16 <-> f32
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// gfx950 converts with one v_cvt_pk_bf16_f32: round to nearest even, NaNs quieted.  This is the
// integer rounding torch applies (bits + 0x7fff + lsb, NaN -> quiet NaN) for every one of the 2^32
// inputs, denormals included.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Workgroup barrier that orders LDS only: each wave waits for its own LDS operations, not for its
// outstanding global loads and stores (which __syncthreads' workgroup fence would drain).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Two floats rounded to bf16 and packed low / high into one dword (a single conversion).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Round a float to the nearest value of the storage dtype (identity for f32).  bf16: one
// v_cvt_pk_bf16_f32 with f in the high half and 0 in the low half leaves the rounded value's float32
// bit pattern in the register itself (no shift back).
template <int DT>
__device__ __forceinline__ float rnd(float f) {
  if constexpr (DT == kBF16) {
    return __uint_as_float(pack_bf16x2(0.0f, f));
  } else {
    return f;
  }
}

template <int DT>
struct Elem;
template <>
struct Elem<kF32> {
  using T = float;
};
template <>
struct Elem<kBF16> {
  using T = uint16_t;
};

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (DT == kBF16) {
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  } else {
    return static_cast<const float*>(p)[i];
  }
}

template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  if constexpr (DT == kBF16) {
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  } else {
    static_cast<float*>(p)[i] = v;
  }
}

// Raw bits of one element: bf16 zero-extended, f32 as is.  Kernels that issue their loads early keep
// the bits and convert where the value is used (from_bits), so no conversion forces a wait for the
// load right after it is issued.
template <int DT>
__device__ __forceinline__ uint32_t ld_bits(const void* p, int64_t i) {
  if constexpr (DT == kBF16)
    return static_cast<const uint16_t*>(p)[i];
  else
    return static_cast<const uint32_t*>(p)[i];
}
template <int DT>
__device__ __forceinline__ float from_bits(uint32_t b) {
  return __uint_as_float(DT == kBF16 ? b << 16 : b);
}

// acc + a * b where the product of a and b is exact in float32 (values of the bf16 layer dtype: 8-bit
// significands): one fused multiply-add then gives the bits of the separate multiply and add, which is what
// float32 operands keep (the library is built with -ffp-contract=off).
template <int DT>
__device__ __forceinline__ float madd(float a, float b, float acc) {
  if constexpr (DT == kBF16)
    return __builtin_fmaf(a, b, acc);
  else
    return acc + a * b;
}

// Four consecutive elements at p[i .. i+3] in one store; needs i*size 8-byte (bf16) / 16-byte (f32) aligned.
template <int DT>
__device__ __forceinline__ void st4(void* p, int64_t i, const float (&v)[4]) {
  if constexpr (DT == kBF16) {
    const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
    const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
    *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p) + i) = make_uint2(lo, hi);
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
  }
}

// ---------------------------------------------------------------------------
// Branch-free float32 transcendentals for the gates (a few ulp; every result that the reference
// rounds to bf16 is rounded again afterwards).  Built on the hardware exp2 / reciprocal.
// ---------------------------------------------------------------------------
// e^x = 2^(x log2 e), with x * log2 e split into a rounded product and its error term so that
// the argument error stays below an ulp of 2^t for |x| up to ~88.
__device__ __forceinline__ float fast_exp(float x) {
  constexpr float kL2e = 1.44269504088896340736f;
  const float t = x * kL2e;
  const float err = __builtin_fmaf(x, kL2e, -t) + x * 1.925963033500e-8f;  // log2(e) - kL2e
  const float r = __builtin_amdgcn_exp2f(t);
  return __builtin_fmaf(r, err * 0.69314718055994531f, r);
}

// 1 / (1 + e^-x); saturates to 0 / 1 without NaN for large |x|.
__device__ __forceinline__ float sigmoidf_(float x) { return __builtin_amdgcn_rcpf(1.0f + fast_exp(-x)); }

// tanh: odd Taylor polynomial below |x| = 0.25 (truncation < 1e-8 relative), otherwise
// sign(x) * (1 - 2 / (e^{2|x|} + 1)).
__device__ __forceinline__ float tanhf_(float x) {
  const float ax = fabsf(x);
  const float big = 1.0f - 2.0f * __builtin_amdgcn_rcpf(fast_exp(2.0f * ax) + 1.0f);
  const float x2 = x * x;
  float p = __builtin_fmaf(x2, 62.0f / 2835.0f, -17.0f / 315.0f);
  p = __builtin_fmaf(x2, p, 2.0f / 15.0f);
  p = __builtin_fmaf(x2, p, -1.0f / 3.0f);
  const float small = __builtin_fmaf(x * x2, p, x);
  return ax < 0.25f ? small : __builtin_copysignf(big, x);
}

// ---------------------------------------------------------------------------
// per-token int8 activation quantization (reference tesm.py:206-209)
//   scale = 127 / max(amax, eps), evaluated by torch as reciprocal() * 127
//   code  = clamp(rne(x * scale), -128, 127)
// with every op rounded to the activation dtype.
// ---------------------------------------------------------------------------
template <int DT>
__device__ __forceinline__ float act_scale(float amax, float eps) {
  if constexpr (DT == kBF16) {
    const float e = rnd<DT>(eps);
    const float d = amax < e ? e : amax;
    return rnd<DT>(rnd<DT>(1.0f / d) * 127.0f);
  } else {
    const float d = amax < eps ? eps : amax;
    return (1.0f / d) * 127.0f;
  }
}

template <int DT>
__device__ __forceinline__ int act_code(float v, float scale) {
  float r = rintf(rnd<DT>(v * scale));
  r = fminf(fmaxf(r, -128.0f), 127.0f);
  return static_cast<int>(r);
}

// Byte position of code e (0..15) inside its 16-code group in "layout 1", the order the INT2
// products read: byte 4s + j holds code 4j + s.
__device__ __forceinline__ int layout1_pos(int e) { return 4 * (e & 3) + (e >> 2); }

// ---------------------------------------------------------------------------
// Per-token activation quantization of one 16-code group (shared by quant_act and the fused
// decode-size product)
// ---------------------------------------------------------------------------
// Load the 16 values of code group g (codes 16g..16g+15) of one row, zero past K.
template <int DT, bool VEC>
__device__ __forceinline__ void load_group(const void* __restrict__ x, int64_t base, int64_t K, int64_t g,
                                           float (&v)[16]) {
  const int64_t k0 = g * 16;
  if (VEC && k0 + 16 <= K) {
    if constexpr (DT == kBF16) {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + base + k0);
      const uint4 a = p[0], b = p[1];
      const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      }
    } else {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(x) + base + k0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 f = p[i];
        v[4 * i] = f.x;
        v[4 * i + 1] = f.y;
        v[4 * i + 2] = f.z;
        v[4 * i + 3] = f.w;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (k0 + i < K) ? ld<DT>(x, base + k0 + i) : 0.0f;
  }
}

// A lane's G groups of 16 elements (groups g0, g0 + LPR, ...) of a row starting at element `base`,
// for 16-byte aligned rows with K % 16 == 0: every group's 16-byte loads are issued in straight-line
// code before the first is converted, so the lane waits for memory once.  Groups past K re-read the
// row's last group and come back as zeros.
template <int DT, int G, int LPR>
__device__ __forceinline__ void load_groups(const void* __restrict__ x, int64_t base, int64_t K, int64_t g0,
                                            float (&v)[G][16]) {
  constexpr int ES = DT == kBF16 ? 2 : 4, NV = 16 * ES / 16;  // 16-byte loads per group
  const int64_t nfull = K / 16;
  const char* xr = static_cast<const char*>(x) + base * ES;
  uint4 raw[G][NV];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    const int64_t g = g0 + LPR * gi, gl = g < nfull ? g : nfull - 1;
    const uint4* p = reinterpret_cast<const uint4*>(xr + gl * 16 * ES);
#pragma unroll
    for (int q = 0; q < NV; ++q) raw[gi][q] = p[q];
  }
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    const bool in = g0 + LPR * gi < nfull;
    uint32_t wd[4 * NV];  // the group's words, zero past K (one select per word rather than per value)
#pragma unroll
    for (int q = 0; q < NV; ++q) {
      wd[4 * q] = in ? raw[gi][q].x : 0u;
      wd[4 * q + 1] = in ? raw[gi][q].y : 0u;
      wd[4 * q + 2] = in ? raw[gi][q].z : 0u;
      wd[4 * q + 3] = in ? raw[gi][q].w : 0u;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[gi][i] = DT == kBF16 ? __uint_as_float(i % 2 == 0 ? wd[i / 2] << 16 : wd[i / 2] & 0xffff0000u)
                             : __uint_as_float(wd[i]);
  }
}

// Byte 0 of each of four words, gathered into one word (b0 lowest) by three v_perm_b32.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);  // b0.0, b1.0, 0, 0
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);  // b2.0, b3.0, 0, 0
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

// Codes of one group, packed in the requested layout; adds the codes to rs.  Each code is act_code's
// clamp(rne(rnd(x * sc)), -128, 127) formed as clamp first (the bounds are integers, so clamping before or
// after the rounding agrees; NaN gives -128 either way), then + 1.5 * 2^23: the addition rounds the value
// to an integer, nearest even, held in the low mantissa bits, so the low byte of the sum's bits is the code
// in two's complement.  The bytes are gathered by v_perm_b32 and summed by a four-byte dot product.
template <int DT>
__device__ __forceinline__ uint4 group_codes(const float (&v)[16], float sc, int layout, int32_t& rs) {
  uint32_t c[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float t = fminf(fmaxf(rnd<DT>(v[i] * sc), -128.0f), 127.0f);
    c[i] = __float_as_uint(t + 12582912.0f);
  }
  uint4 out;
  if (layout == 1) {
    out.x = pack_low_bytes(c[0], c[4], c[8], c[12]);
    out.y = pack_low_bytes(c[1], c[5], c[9], c[13]);
    out.z = pack_low_bytes(c[2], c[6], c[10], c[14]);
    out.w = pack_low_bytes(c[3], c[7], c[11], c[15]);
  } else {
    out.x = pack_low_bytes(c[0], c[1], c[2], c[3]);
    out.y = pack_low_bytes(c[4], c[5], c[6], c[7]);
    out.z = pack_low_bytes(c[8], c[9], c[10], c[11]);
    out.w = pack_low_bytes(c[12], c[13], c[14], c[15]);
  }
  rs = __builtin_amdgcn_sdot4(static_cast<int>(out.x), 0x01010101, rs, false);
  rs = __builtin_amdgcn_sdot4(static_cast<int>(out.y), 0x01010101, rs, false);
  rs = __builtin_amdgcn_sdot4(static_cast<int>(out.z), 0x01010101, rs, false);
  rs = __builtin_amdgcn_sdot4(static_cast<int>(out.w), 0x01010101, rs, false);
  return out;
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------
// Lane exchanges for order-free reductions inside groups of WIDTH lanes: DPP quad permutes (lane ^ 1,
// lane ^ 2), the half-row and row mirrors (a lane of the other 4- and 8-lane group, which is all a
// butterfly needs once each group's lanes agree), a swizzle (lane ^ 16 within 32 lanes), and for the
// whole wave the two half-wave results read from lanes 0 and 32 (v_readlane: a uniform total).  DPP
// moves and lane reads are VALU operations; only the swizzle goes through the LDS crossbar, where
// every __shfl_xor step would.  Full-wave reductions need every lane active.
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1, 0, 3, 2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2, 3, 0, 1]
constexpr int kDppHalfMirror = 0x141;  // lane i <- 7 - i within 8
constexpr int kDppMirror = 0x140;      // lane i <- 15 - i within 16
constexpr int kSwzXor16 = 0x401F;      // ds_swizzle bit mode: and 0x1f, or 0, xor 0x10

template <int WIDTH = 64>
__device__ __forceinline__ float wave_max(float v) {
  if constexpr (WIDTH >= 2) v = fmaxf(v, __int_as_float(dpp_mov<kDppXor1>(__float_as_int(v))));
  if constexpr (WIDTH >= 4) v = fmaxf(v, __int_as_float(dpp_mov<kDppXor2>(__float_as_int(v))));
  if constexpr (WIDTH >= 8) v = fmaxf(v, __int_as_float(dpp_mov<kDppHalfMirror>(__float_as_int(v))));
  if constexpr (WIDTH >= 16) v = fmaxf(v, __int_as_float(dpp_mov<kDppMirror>(__float_as_int(v))));
  if constexpr (WIDTH >= 32) v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), kSwzXor16)));
  if constexpr (WIDTH >= 64)  // the two half-wave maxima, read from lanes 0 and 32
    v = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
  return v;
}

template <int WIDTH = 64>
__device__ __forceinline__ int wave_sum_i(int v) {
  if constexpr (WIDTH >= 2) v += dpp_mov<kDppXor1>(v);
  if constexpr (WIDTH >= 4) v += dpp_mov<kDppXor2>(v);
  if constexpr (WIDTH >= 8) v += dpp_mov<kDppHalfMirror>(v);
  if constexpr (WIDTH >= 16) v += dpp_mov<kDppMirror>(v);
  if constexpr (WIDTH >= 32) v += __builtin_amdgcn_ds_swizzle(v, kSwzXor16);
  if constexpr (WIDTH >= 64) v = __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 32);
  return v;
}

template <int WIDTH = 64>
__device__ __forceinline__ float wave_sum_f(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, WIDTH);
  return v;
}

// Float sums of N values over the whole wave on wave_sum_i's exchanges (four DPP steps, the swizzle),
// the two half-wave totals then read from lanes 0 and 32 and added: every lane receives each total.
// The N chains are independent, so their exchanges overlap.  The addition tree differs from
// wave_sum_f's butterfly: a kernel keeps one of the two wherever its sums must match another's.
template <int N>
__device__ __forceinline__ void wave_sum_fn(float (&v)[N]) {
#pragma unroll
  for (int n = 0; n < N; ++n) v[n] += __int_as_float(dpp_mov<kDppXor1>(__float_as_int(v[n])));
#pragma unroll
  for (int n = 0; n < N; ++n) v[n] += __int_as_float(dpp_mov<kDppXor2>(__float_as_int(v[n])));
#pragma unroll
  for (int n = 0; n < N; ++n) v[n] += __int_as_float(dpp_mov<kDppHalfMirror>(__float_as_int(v[n])));
#pragma unroll
  for (int n = 0; n < N; ++n) v[n] += __int_as_float(dpp_mov<kDppMirror>(__float_as_int(v[n])));
#pragma unroll
  for (int n = 0; n < N; ++n) v[n] += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v[n]), kSwzXor16));
#pragma unroll
  for (int n = 0; n < N; ++n)
    v[n] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[n]), 0)) +
           __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[n]), 32));
}

template <int WIDTH = 64>
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
  for (int m = WIDTH / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, WIDTH);
  return v;
}

// ---------------------------------------------------------------------------
// host-side error plumbing (thread-local last error, returned codes)
// ---------------------------------------------------------------------------
enum Status : int {
  kOk = 0,
  kErrInvalidArg = 1,
  kErrAlignment = 2,
  kErrUnsupported = 3,
  kErrLaunch = 4,
  kErrWorkspace = 5,
};

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int check_launch(const char* what);

// Launch log: while enabled (tesm_hip_launch_log), every kernel launch appends the kernel's name
// with its template arguments (the runtime's name of the kernel's host stub, demangled).  The launch
// sites pass their stream through TESM_LOGGED, so a disabled log costs one relaxed load per launch.
extern int g_launch_log_on;
void log_kernel(const void* host_stub);
template <auto K>
inline void note_kernel() {
  if (__atomic_load_n(&g_launch_log_on, __ATOMIC_RELAXED)) log_kernel(reinterpret_cast<const void*>(K));
}

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }
inline bool aligned(const void* p, int64_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// K padding used by every int8-code and packed-INT2 buffer of the BitLinear path:
// one GEMM K tile is 128 codes.
constexpr int64_t kKTile = 128;
inline int64_t kpad(int64_t K) { return round_up(K < 1 ? 1 : K, kKTile); }

}  // namespace tesm

#define TESM_REQUIRE(cond, code, msg)        \
  do {                                       \
    if (!(cond)) return ::tesm::fail((code), (msg)); \
  } while (0)

// Stream argument of a kernel launch that also records the kernel in the launch log:
//   kern<A, B><<<grid, block, lds, TESM_LOGGED(st, kern<A, B>)>>>(args);
#define TESM_LOGGED(st, ...) (::tesm::note_kernel<&__VA_ARGS__>(), (st))
