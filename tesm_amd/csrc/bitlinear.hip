// INT2 x INT8 BitLinear products for gfx950.
//
// Reference semantics (tesm_ssm/modules/tesm.py:238-290, torch branch):
//   y = F.linear(q_x / s_x, q_w / s_w) with q_x int8 per-token codes and q_w ternary codes.
// Here the contraction is done exactly in int32 on the codes and scaled once:
//   acc = sum_k q_x[m,k] * q_w[n,k];   y = acc / s_x[m] * c_w     (c_w = 1 / s_w rounded)
// Weights arrive packed (code + 1 in {0,1,2}, four per byte), so the kernels form
//   acc = sum_k q_x * u_w - sum_k q_x      (u = code + 1)
// and the per-row sum of activation codes (from the quantization kernel) removes the offset.
//
// Two kernels:
//   * gemv_kernel  (M <= 4): bandwidth-bound decode path.  Each lane streams 16-byte packed
//     chunks (64 codes) with one 128-bit load, unpacks in registers with shift/and and
//     multiplies with v_dot4_i32_i8 against activation codes held in registers.
//   * mfma_kernel  (M > 4): LDS-tiled int8 MFMA (v_mfma_i32_16x16x64_i8).  Packed weight tiles
//     are unpacked to int8 while being staged in LDS; A and B fragments are stored in MFMA
//     lane order so every ds_read_b128 of a wave is one contiguous 1 KiB block.
#include "tesm_hip_internal.h"

namespace tesm {

namespace {

__device__ __forceinline__ uint32_t unpack_u(uint32_t w, int s) { return (w >> (2 * s)) & 0x03030303u; }

template <int OUT_DT>
__device__ __forceinline__ void store_plain(const LinearArgs& a, int64_t m, int64_t n, float v) {
  if (a.bias) v = v + ld<OUT_DT>(a.bias, n);
  st<OUT_DT>(a.out, m * a.ldo + n, v);
}

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
template <int LPR, int MR, int NCH, int OUT_DT>
__global__ __launch_bounds__(256) void gemv_kernel(LinearArgs a) {
  constexpr int RPG = 4;          // output rows per lane group (independent loads in flight)
  constexpr int GPW = 64 / LPR;   // lane groups per wave
  const LinearOperand& o = a.op[0];
  const int lane = threadIdx.x & 63;
  const int g = lane & (LPR - 1);
  const int64_t group = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * GPW + lane / LPR;
  const int64_t n0 = group * RPG;
  if (n0 >= a.N) return;
  const int64_t nch = a.Kp / 64;

  // unconditional loads from clamped rows / chunks (masked afterwards): all in flight at once
  uint4 W[RPG][NCH];
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    const int64_t n = n0 + r;
    const int64_t nc = n < a.N ? n : a.N - 1;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int64_t c = g + LPR * i;
      const int64_t cc = c < nch ? c : nch - 1;
      // rows past N only feed outputs that are never stored; chunks past the row are masked at use
      W[r][i] = *reinterpret_cast<const uint4*>(o.w + nc * o.ldw + 16 * cc);
    }
  }
  uint32_t X[MR][NCH][16];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int64_t mc = m < a.M ? m : a.M - 1;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int64_t c = g + LPR * i;
      const int64_t cc = c < nch ? c : nch - 1;
#pragma unroll
      for (int d = 0; d < 4; ++d) {
        const uint4 v = *reinterpret_cast<const uint4*>(o.q + mc * o.ldq + 64 * cc + 16 * d);
        X[m][i][4 * d + 0] = v.x;
        X[m][i][4 * d + 1] = v.y;
        X[m][i][4 * d + 2] = v.z;
        X[m][i][4 * d + 3] = v.w;
      }
    }
  }
  int acc[RPG][MR];
#pragma unroll
  for (int r = 0; r < RPG; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0;

#pragma unroll
  for (int r = 0; r < RPG; ++r) {
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      // a lane's chunk past the end of the row contributes nothing (code 0 everywhere)
      const bool live = g + LPR * i < nch;
      const uint32_t wd[4] = {live ? W[r][i].x : 0u, live ? W[r][i].y : 0u, live ? W[r][i].z : 0u,
                              live ? W[r][i].w : 0u};
#pragma unroll
      for (int d = 0; d < 4; ++d) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int u = static_cast<int>(unpack_u(wd[d], s));
#pragma unroll
          for (int m = 0; m < MR; ++m)
            acc[r][m] = __builtin_amdgcn_sdot4(u, static_cast<int>(X[m][i][4 * d + s]), acc[r][m], false);
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RPG; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      int v = acc[r][m];
#pragma unroll
      for (int mask = LPR / 2; mask > 0; mask >>= 1) v += __shfl_xor(v, mask, 64);
      acc[r][m] = v;
    }
  if (g != 0) return;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= a.M) break;
    const float inv = 1.0f / o.s_x[m];
    const int32_t rs = o.rowsum[m];
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
      const int64_t n = n0 + r;
      if (n >= a.N) break;
      const int32_t av = acc[r][m] - rs;
      if (a.acc_dump) a.acc_dump[m * a.N + n] = av;
      const float cw = o.c_w_per_row ? o.c_w[n] : o.c_w[0];
      store_plain<OUT_DT>(a, m, n, (static_cast<float>(av) * inv) * cw);
    }
  }
}

// ---------------------------------------------------------------------------
// MFMA GEMM
// ---------------------------------------------------------------------------
template <int WM, int WN, int TM, int TN>
struct Cfg {
  static constexpr int NT = WM * WN * 64;
  static constexpr int BM = WM * TM * 16, BN = WN * TN * 16, BK = 128;
  static constexpr int A_BYTES = BM * BK;        // int8 codes, fragment order
  static constexpr int B_BYTES = BN * BK / 4;    // packed INT2, fragment order (one dword per lane)
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_CHUNKS = BM * BK / 16;  // 16-byte code chunks per K tile
  static constexpr int B_CHUNKS = BN * BK / 64;  // 16-byte packed chunks per K tile
  static constexpr int A_PT = (A_CHUNKS + NT - 1) / NT;
  static constexpr int B_PT = (B_CHUNKS + NT - 1) / NT;
};

// LDS fragment order.  A: fragment (tile t of 16 rows, k-step ks of 64 codes) is 1 KiB; lane L holds
// the 16 code bytes of row 16t + L%16, code group 4ks + L/16.  B: fragment (tile t of 16 columns,
// ks) is 256 bytes; lane L holds the packed dword (16 codes) of column 16t + L%16, group 4ks + L/16.
// Lane L's A and B operands therefore cover the same 16 codes, in the order the unpack produces.
__device__ __forceinline__ int a_frag_off(int r, int kg) {
  return (((r >> 4) * 2 + (kg >> 2)) << 10) + (((r & 15) + 16 * (kg & 3)) << 4);
}
__device__ __forceinline__ int b_frag_off(int r, int kg) {
  return (((r >> 4) * 2 + (kg >> 2)) << 8) + (((r & 15) + 16 * (kg & 3)) << 2);
}

__device__ __forceinline__ v4i unpack_frag(uint32_t w) {
  return v4i{static_cast<int>(unpack_u(w, 0)), static_cast<int>(unpack_u(w, 1)), static_cast<int>(unpack_u(w, 2)),
             static_cast<int>(unpack_u(w, 3))};
}

template <class C>
__device__ __forceinline__ void gemm_gload(const int8_t* const (&pa)[C::A_PT], const uint8_t* const (&pb)[C::B_PT],
                                           const bool (&vb)[C::B_PT], int64_t k0, v4i (&ra)[C::A_PT],
                                           v4i (&rb)[C::B_PT]) {
#pragma unroll
  for (int p = 0; p < C::A_PT; ++p) ra[p] = *reinterpret_cast<const v4i*>(pa[p] + k0);
#pragma unroll
  for (int p = 0; p < C::B_PT; ++p)
    if (vb[p]) rb[p] = *reinterpret_cast<const v4i*>(pb[p] + k0 / 4);
}

// dword d of a packed B chunk is code group 4h + d, which sits 16 lanes (64 bytes) further on in
// the fragment
template <class C>
__device__ __forceinline__ void gemm_sstore(const int (&la)[C::A_PT], const int (&lb)[C::B_PT],
                                            const bool (&vb)[C::B_PT], const v4i (&ra)[C::A_PT],
                                            const v4i (&rb)[C::B_PT], char* stage) {
#pragma unroll
  for (int p = 0; p < C::A_PT; ++p) *reinterpret_cast<v4i*>(stage + la[p]) = ra[p];
#pragma unroll
  for (int p = 0; p < C::B_PT; ++p) {
    if (vb[p]) {
      *reinterpret_cast<int*>(stage + lb[p]) = rb[p].x;
      *reinterpret_cast<int*>(stage + lb[p] + 64) = rb[p].y;
      *reinterpret_cast<int*>(stage + lb[p] + 128) = rb[p].z;
      *reinterpret_cast<int*>(stage + lb[p] + 192) = rb[p].w;
    }
  }
}

template <class C, int WN, int TM, int TN>
__device__ __forceinline__ void mfma_mainloop(const LinearOperand& o, int64_t M, int64_t N, int64_t m0, int64_t n0,
                                              int64_t Kp, v4i (&acc)[TM][TN], char* smem) {
  const int t = threadIdx.x;
  __builtin_assume(t < C::NT);
  const int lane = t & 63, w = t >> 6;
  const int wm = w / WN, wn = w % WN;
  constexpr bool kAllB = (C::B_CHUNKS % C::NT) == 0;

  // per-chunk global sources and LDS destinations; rows past M / columns past N read the last
  // valid one and only feed accumulator entries that are never stored
  const int8_t* pa[C::A_PT];
  int la[C::A_PT];
#pragma unroll
  for (int p = 0; p < C::A_PT; ++p) {
    const int c = t + p * C::NT;
    const int64_t m = m0 + (c >> 3);
    pa[p] = o.q + (m < M ? m : M - 1) * o.ldq + 16 * (c & 7);
    la[p] = a_frag_off(c >> 3, c & 7);
  }
  const uint8_t* pb[C::B_PT];
  int lb[C::B_PT];
  bool vb[C::B_PT];
#pragma unroll
  for (int p = 0; p < C::B_PT; ++p) {
    const int c = t + p * C::NT;
    vb[p] = kAllB || c < C::B_CHUNKS;
    const int64_t n = n0 + (c >> 1);
    pb[p] = o.w + (n < N ? n : N - 1) * o.ldw + 16 * (c & 1);
    lb[p] = C::A_BYTES + b_frag_off(c >> 1, 4 * (c & 1));
  }
  v4i ra[C::A_PT], rb[C::B_PT];
  const int64_t nk = Kp / C::BK;
  gemm_gload<C>(pa, pb, vb, 0, ra, rb);
  gemm_sstore<C>(la, lb, vb, ra, rb, smem);
  __syncthreads();
  for (int64_t kt = 0; kt < nk; ++kt) {
    const char* cur = smem + (kt & 1) * C::STAGE;
    const bool more = kt + 1 < nk;
    if (more) gemm_gload<C>(pa, pb, vb, (kt + 1) * C::BK, ra, rb);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v4i af[TM];
      uint32_t bw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const v4i*>(cur + (((wm * TM + i) * 2 + ks) << 10) + lane * 16);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bw[j] = *reinterpret_cast<const uint32_t*>(cur + C::A_BYTES + (((wn * TN + j) * 2 + ks) << 8) + lane * 4);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const v4i bf = unpack_frag(bw[j]);
        // weights as the MFMA's A operand: the accumulator comes out transposed, so each lane holds
        // 4 consecutive output columns of one row (vector stores in the epilogue)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af[i], acc[i][j], 0, 0, 0);
      }
    }
    if (more) gemm_sstore<C>(la, lb, vb, ra, rb, smem + ((kt + 1) & 1) * C::STAGE);
    __syncthreads();
  }
}

// Tile order for a 1-D grid: workgroups are handed to the 8 XCDs round-robin by id, so id is
// mapped to a tile such that each XCD gets a contiguous run of tiles (row-major over
// (M tile, N tile)); consecutive tiles of one XCD share A rows in that XCD's L2.
__device__ __forceinline__ void xcd_tile(int64_t ntm, int64_t ntn, int64_t& tm, int64_t& tn) {
  constexpr int64_t kXcd = 8;
  const int64_t total = ntm * ntn, pid = blockIdx.x;
  const int64_t x = pid % kXcd, i = pid / kXcd;
  const int64_t q = total / kXcd, r = total % kXcd;
  const int64_t tile = x * q + (x < r ? x : r) + i;
  tm = tile / ntn;
  tn = tile - tm * ntn;
}

// With the weights as the A operand, element r of lane L's accumulator is output row L%16 and
// output column 4*(L/16) + r of the 16 x 16 tile.
template <int OUT_DT>
__device__ __forceinline__ void store4(void* out, int64_t idx, const float (&v)[4], bool vec) {
  if (vec) {
    if constexpr (OUT_DT == kBF16) {
      const uint32_t lo = static_cast<uint32_t>(f32_to_bf16(v[0])) | (static_cast<uint32_t>(f32_to_bf16(v[1])) << 16);
      const uint32_t hi = static_cast<uint32_t>(f32_to_bf16(v[2])) | (static_cast<uint32_t>(f32_to_bf16(v[3])) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + idx) = make_uint2(lo, hi);
    } else {
      *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = make_float4(v[0], v[1], v[2], v[3]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) st<OUT_DT>(out, idx + r, v[r]);
  }
}

template <int DT>
__device__ __forceinline__ void load4(const void* p, int64_t idx, bool vec, float (&v)[4]) {
  if (vec) {
    if constexpr (DT == kBF16) {
      const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + idx);
      v[0] = __uint_as_float(w.x << 16);
      v[1] = __uint_as_float(w.x & 0xffff0000u);
      v[2] = __uint_as_float(w.y << 16);
      v[3] = __uint_as_float(w.y & 0xffff0000u);
    } else {
      const float4 f = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + idx);
      v[0] = f.x;
      v[1] = f.y;
      v[2] = f.z;
      v[3] = f.w;
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = ld<DT>(p, idx + r);
  }
}

// 4-element vector access at element (m * ld + n) is aligned for every m and every n % 4 == 0.
template <int DT>
__device__ __forceinline__ bool vec4_ok(const void* p, int64_t ld) {
  constexpr int64_t bytes = DT == kBF16 ? 8 : 16;
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0 && (ld * (DT == kBF16 ? 2 : 4)) % bytes == 0;
}

template <int WM, int WN, int TM, int TN, int EPI, int OUT_DT>
__global__ __launch_bounds__(WM* WN * 64) void mfma_kernel(LinearArgs a) {
  using C = Cfg<WM, WN, TM, TN>;
  __shared__ __attribute__((aligned(16))) char smem[2 * C::STAGE];
  int64_t tm, tn;
  xcd_tile((a.M + C::BM - 1) / C::BM, (a.N + C::BN - 1) / C::BN, tm, tn);
  const int64_t m0 = tm * C::BM;
  const int64_t n0 = tn * C::BN;
  v4i acc0[TM][TN], acc1[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      acc0[i][j] = v4i{0, 0, 0, 0};
      acc1[i][j] = v4i{0, 0, 0, 0};
    }
  mfma_mainloop<C, WN, TM, TN>(a.op[0], a.M, a.N, m0, n0, a.Kp, acc0, smem);
  if constexpr (EPI == kEpiOutputGate) mfma_mainloop<C, WN, TM, TN>(a.op[1], a.M, a.N, m0, n0, a.Kp, acc1, smem);

  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w / WN, wn = w % WN;
  const LinearOperand& o0 = a.op[0];
  const LinearOperand& o1 = a.op[1];
  const bool vout = vec4_ok<OUT_DT>(a.out, a.ldo);
  bool vin = false;
  if constexpr (EPI == kEpiOutputGate) vin = vec4_ok<OUT_DT>(a.local, a.ld_local) && vec4_ok<OUT_DT>(a.gate, a.ld_gate);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + (wm * TM + i) * 16 + (lane & 15);
    if (m >= a.M) continue;
    const float inv0 = 1.0f / o0.s_x[m];
    const int32_t rs0 = o0.rowsum[m];
    float inv1 = 0.0f;
    int32_t rs1 = 0;
    if constexpr (EPI == kEpiOutputGate) {
      inv1 = 1.0f / o1.s_x[m];
      rs1 = o1.rowsum[m];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t nb = n0 + (wn * TN + j) * 16 + 4 * (lane >> 4);
      if (nb >= a.N) continue;
      const bool full = nb + 3 < a.N;
      float v[4], lo[4], gt[4];
      if constexpr (EPI == kEpiOutputGate) {
        if (full) {
          load4<OUT_DT>(a.local, m * a.ld_local + nb, vin, lo);
          load4<OUT_DT>(a.gate, m * a.ld_gate + nb, vin, gt);
        } else {
          for (int r = 0; r < 4; ++r) {
            lo[r] = nb + r < a.N ? ld<OUT_DT>(a.local, m * a.ld_local + nb + r) : 0.0f;
            gt[r] = nb + r < a.N ? ld<OUT_DT>(a.gate, m * a.ld_gate + nb + r) : 0.0f;
          }
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = nb + r;
        v[r] = 0.0f;
        if (n >= a.N) continue;
        const float cw0 = o0.c_w_per_row ? o0.c_w[n] : o0.c_w[0];
        const int32_t a0 = acc0[i][j][r] - rs0;
        if (a.acc_dump) a.acc_dump[m * a.N + n] = a0;
        const float v0 = (static_cast<float>(a0) * inv0) * cw0;
        if constexpr (EPI == kEpiStore) {
          v[r] = a.bias ? v0 + ld<OUT_DT>(a.bias, n) : v0;
        } else {
          const float cw1 = o1.c_w_per_row ? o1.c_w[n] : o1.c_w[0];
          const float sp = rnd<OUT_DT>(v0);
          const float ep = rnd<OUT_DT>((static_cast<float>(acc1[i][j][r] - rs1) * inv1) * cw1);
          const float g = rnd<OUT_DT>(sigmoidf_(gt[r]));
          v[r] = rnd<OUT_DT>(rnd<OUT_DT>(lo[r] + rnd<OUT_DT>(g * sp)) + ep);
        }
      }
      if (full) {
        store4<OUT_DT>(a.out, m * a.ldo + nb, v, vout);
      } else {
        for (int r = 0; r < 4 && nb + r < a.N; ++r) st<OUT_DT>(a.out, m * a.ldo + nb + r, v[r]);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Output gate over whole rows: a workgroup owns 16 rows and all N = d_model columns (4 waves side by
// side, NCT 16-column tiles each), so after y = local + sigmoid(gate)*state_proj + ent_proj it can
// quantize y per token for out_proj without writing y.  Operands stream from global/L2 into
// registers (A: 16 code rows; B: one packed dword per lane per tile), double buffered per k-step.
// ---------------------------------------------------------------------------
template <int NCT, int DT>
__global__ __launch_bounds__(256) void gate_rowq_kernel(LinearArgs a, RowQuant o) {
  extern __shared__ __attribute__((aligned(16))) char lds_rowq[];
  int8_t* codes = reinterpret_cast<int8_t*>(lds_rowq);                              // [16][ldq]
  float* red = reinterpret_cast<float*>(lds_rowq + 16 * o.ldq);                     // [16 rows][4 waves]
  int32_t* redi = reinterpret_cast<int32_t*>(lds_rowq + 16 * o.ldq + 16 * 4 * 4);   // [16 rows][4 waves]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t col0 = static_cast<int64_t>(w) * NCT * 16;
  const LinearOperand& o0 = a.op[0];
  const LinearOperand& o1 = a.op[1];
  const int row = lane & 15;            // the activation row this lane feeds and the output row it holds
  const int64_t m = m0 + row;
  const bool mok = m < a.M;
  const int64_t nks = a.Kp / 64;

  for (int64_t i = tid; i < 16 * o.ldq / 16; i += 256) reinterpret_cast<uint4*>(codes)[i] = make_uint4(0, 0, 0, 0);

  v4i acc0[NCT], acc1[NCT];
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    acc0[j] = v4i{0, 0, 0, 0};
    acc1[j] = v4i{0, 0, 0, 0};
  }
  v4i xa0, xa1, na0, na1;
  uint32_t bw0[NCT], bw1[NCT], nb0[NCT], nb1[NCT];
  // unconditional loads keep every load of a k-step in flight: rows past M / columns past N read
  // the last valid one and only feed accumulator entries that are never used
  const int64_t mc = mok ? m : a.M - 1;
  auto load = [&](int64_t ks, v4i& r0, v4i& r1, uint32_t (&w0)[NCT], uint32_t (&w1)[NCT]) {
    const int64_t ko = 64 * ks + 16 * (lane >> 4);
    r0 = *reinterpret_cast<const v4i*>(o0.q + mc * o0.ldq + ko);
    r1 = *reinterpret_cast<const v4i*>(o1.q + mc * o1.ldq + ko);
#pragma unroll
    for (int j = 0; j < NCT; ++j) {
      const int64_t n = col0 + 16 * j + (lane & 15);
      const int64_t nc = n < a.N ? n : a.N - 1;
      w0[j] = *reinterpret_cast<const uint32_t*>(o0.w + nc * o0.ldw + ko / 4);
      w1[j] = *reinterpret_cast<const uint32_t*>(o1.w + nc * o1.ldw + ko / 4);
    }
  };
  load(0, xa0, xa1, bw0, bw1);
  for (int64_t ks = 0; ks < nks; ++ks) {
    if (ks + 1 < nks) load(ks + 1, na0, na1, nb0, nb1);
#pragma unroll
    for (int j = 0; j < NCT; ++j) {
      acc0[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack_frag(bw0[j]), xa0, acc0[j], 0, 0, 0);
      acc1[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack_frag(bw1[j]), xa1, acc1[j], 0, 0, 0);
    }
    if (ks + 1 < nks) {
      xa0 = na0;
      xa1 = na1;
#pragma unroll
      for (int j = 0; j < NCT; ++j) {
        bw0[j] = nb0[j];
        bw1[j] = nb1[j];
      }
    }
  }

  // epilogue: lane holds row m, columns col0 + 16j + 4*(lane/16) + r
  const float inv0 = mok ? 1.0f / o0.s_x[m] : 0.0f, inv1 = mok ? 1.0f / o1.s_x[m] : 0.0f;
  const int32_t rs0 = mok ? o0.rowsum[m] : 0, rs1 = mok ? o1.rowsum[m] : 0;
  const float cws0 = o0.c_w[0], cws1 = o1.c_w[0];
  const bool vin = vec4_ok<DT>(a.local, a.ld_local) && vec4_ok<DT>(a.gate, a.ld_gate);
  float y[NCT][4];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    const int64_t nb = col0 + 16 * j + 4 * (lane >> 4);
    float lo[4], gt[4];
    const bool full = nb + 3 < a.N;
    if (mok && full) {
      load4<DT>(a.local, m * a.ld_local + nb, vin, lo);
      load4<DT>(a.gate, m * a.ld_gate + nb, vin, gt);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const bool ok = mok && nb + r < a.N;
        lo[r] = ok ? ld<DT>(a.local, m * a.ld_local + nb + r) : 0.0f;
        gt[r] = ok ? ld<DT>(a.gate, m * a.ld_gate + nb + r) : 0.0f;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = nb + r;
      y[j][r] = 0.0f;
      if (!mok || n >= a.N) continue;
      const float cw0 = o0.c_w_per_row ? o0.c_w[n] : cws0;
      const float cw1 = o1.c_w_per_row ? o1.c_w[n] : cws1;
      const float sp = rnd<DT>((static_cast<float>(acc0[j][r] - rs0) * inv0) * cw0);
      const float ep = rnd<DT>((static_cast<float>(acc1[j][r] - rs1) * inv1) * cw1);
      const float g = rnd<DT>(sigmoidf_(gt[r]));
      const float v = rnd<DT>(rnd<DT>(lo[r] + rnd<DT>(g * sp)) + ep);
      y[j][r] = v;
      mx = fmaxf(mx, fabsf(v));
    }
    if (o.y && mok) {
      if (full) {
        store4<DT>(o.y, m * o.ldy + nb, y[j], vec4_ok<DT>(o.y, o.ldy));
      } else {
        for (int r = 0; r < 4 && nb + r < a.N; ++r) st<DT>(o.y, m * o.ldy + nb + r, y[j][r]);
      }
    }
  }
  // row max over the 4 lanes sharing the row, then over the 4 waves
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (lane < 16) red[row * 4 + w] = mx;
  __syncthreads();
  const float* rr = red + row * 4;
  const float sc = act_scale<DT>(fmaxf(fmaxf(rr[0], rr[1]), fmaxf(rr[2], rr[3])), o.eps);
  int sum = 0;
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = col0 + 16 * j + 4 * (lane >> 4) + r;
      if (!mok || n >= a.N) continue;
      const int q = act_code<DT>(y[j][r], sc);
      // layout 1: element e = n % 16 = 4 * (lane / 16) + r sits at byte 4 * r + lane / 16 of its group
      codes[row * o.ldq + (n & ~static_cast<int64_t>(15)) + 4 * r + (lane >> 4)] = static_cast<int8_t>(q);
      sum += q;
    }
  }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  if (lane < 16) redi[row * 4 + w] = sum;
  __syncthreads();
  if (tid < 16 && m0 + tid < a.M) {
    const int32_t* ri = redi + tid * 4;
    const float* rm = red + tid * 4;
    o.s[m0 + tid] = act_scale<DT>(fmaxf(fmaxf(rm[0], rm[1]), fmaxf(rm[2], rm[3])), o.eps);
    o.rs[m0 + tid] = (ri[0] + ri[1]) + (ri[2] + ri[3]);
  }
  const int64_t chunks = o.ldq / 16;
  for (int r = w; r < 16; r += 4) {
    if (m0 + r >= a.M) continue;
    for (int64_t ck = lane; ck < chunks; ck += 64)
      reinterpret_cast<uint4*>(o.q + (m0 + r) * o.ldq)[ck] = reinterpret_cast<const uint4*>(codes + r * o.ldq)[ck];
  }
}

template <int WM, int WN, int TM, int TN, int EPI>
int run_mfma(const LinearArgs& a, hipStream_t st) {
  using C = Cfg<WM, WN, TM, TN>;
  const int64_t tiles = ((a.N + C::BN - 1) / C::BN) * ((a.M + C::BM - 1) / C::BM);
  TESM_REQUIRE(tiles <= 0x7fffffff, kErrUnsupported, "bitlinear: too many tiles");
  const unsigned grid = static_cast<unsigned>(tiles);
  if (a.out_dt == kBF16)
    mfma_kernel<WM, WN, TM, TN, EPI, kBF16><<<grid, C::NT, 0, st>>>(a);
  else
    mfma_kernel<WM, WN, TM, TN, EPI, kF32><<<grid, C::NT, 0, st>>>(a);
  return check_launch("bitlinear mfma");
}

template <int NCT>
int run_rowq(const LinearArgs& a, const RowQuant& o, hipStream_t st) {
  const size_t lds = static_cast<size_t>(16 * o.ldq + 2 * 16 * 4 * 4);
  const unsigned grid = static_cast<unsigned>((a.M + 15) / 16);
  if (a.out_dt == kBF16)
    gate_rowq_kernel<NCT, kBF16><<<grid, 256, lds, st>>>(a, o);
  else
    gate_rowq_kernel<NCT, kF32><<<grid, 256, lds, st>>>(a, o);
  return check_launch("output gate rowq");
}

template <int LPR, int MR, int NCH>
int run_gemv(const LinearArgs& a, hipStream_t st) {
  constexpr int GPW = 64 / LPR;
  const int64_t groups = (a.N + 3) / 4;
  const int64_t waves = (groups + GPW - 1) / GPW;
  const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
  if (a.out_dt == kBF16)
    gemv_kernel<LPR, MR, NCH, kBF16><<<blocks, 256, 0, st>>>(a);
  else
    gemv_kernel<LPR, MR, NCH, kF32><<<blocks, 256, 0, st>>>(a);
  return check_launch("bitlinear gemv");
}

template <int MR>
int dispatch_gemv(const LinearArgs& a, int64_t nch, hipStream_t st) {
  if (nch <= 4) return run_gemv<4, MR, 1>(a, st);
  if (nch <= 8) return run_gemv<8, MR, 1>(a, st);
  if (nch <= 16) return run_gemv<16, MR, 1>(a, st);
  if (nch <= 32) return run_gemv<32, MR, 1>(a, st);
  if (nch <= 64) return run_gemv<64, MR, 1>(a, st);
  if (nch <= 128) return run_gemv<64, MR, 2>(a, st);
  return run_gemv<64, MR, 4>(a, st);
}

int check_operand(const LinearOperand& o, int64_t Kp, const char* which) {
  std::string p = std::string("bitlinear ") + which + ": ";
  TESM_REQUIRE(o.q && o.s_x && o.rowsum && o.w && o.c_w, kErrInvalidArg, p + "null pointer");
  TESM_REQUIRE(o.ldq >= Kp && o.ldq % 16 == 0, kErrInvalidArg, p + "ldq must be >= Kp and a multiple of 16");
  TESM_REQUIRE(o.ldw >= Kp / 4 && o.ldw % 16 == 0, kErrInvalidArg, p + "ldw must be >= Kp/4 and a multiple of 16");
  TESM_REQUIRE(aligned(o.q, 16) && aligned(o.w, 16), kErrAlignment, p + "codes and packed weights must be 16-byte aligned");
  return kOk;
}

}  // namespace

int launch_linear(const LinearArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.M >= 0 && a.N >= 0, kErrInvalidArg, "bitlinear: negative size");
  TESM_REQUIRE(a.Kp >= kKTile && a.Kp % kKTile == 0, kErrInvalidArg, "bitlinear: Kp must be a positive multiple of 128");
  TESM_REQUIRE(a.out_dt == kF32 || a.out_dt == kBF16, kErrInvalidArg, "bitlinear: out dtype must be 0 or 1");
  TESM_REQUIRE(a.epilogue == kEpiStore || a.epilogue == kEpiOutputGate, kErrInvalidArg, "bitlinear: bad epilogue");
  if (a.M == 0 || a.N == 0) return kOk;
  TESM_REQUIRE(a.out && a.ldo >= a.N, kErrInvalidArg, "bitlinear: need out and ldo >= N");
  if (int rc = check_operand(a.op[0], a.Kp, "op0")) return rc;
  if (a.epilogue == kEpiOutputGate) {
    if (int rc = check_operand(a.op[1], a.Kp, "op1")) return rc;
    TESM_REQUIRE(a.local && a.gate && a.ld_local >= a.N && a.ld_gate >= a.N, kErrInvalidArg,
                 "bitlinear output gate: need local and gate operands");
    TESM_REQUIRE(a.bias == nullptr, kErrInvalidArg, "bitlinear output gate: bias unsupported");
  }
  const int64_t nch = a.Kp / 64;
  if (a.epilogue == kEpiStore && a.M <= 4 && nch <= 256) {
    if (a.M == 1) return dispatch_gemv<1>(a, nch, st);
    if (a.M == 2) return dispatch_gemv<2>(a, nch, st);
    return dispatch_gemv<4>(a, nch, st);
  }
  if (a.epilogue == kEpiStore) {
    if (a.M <= 32) return run_mfma<1, 4, 2, 1, kEpiStore>(a, st);
    // 64x128 tiles with the four waves along N: measured fastest for M >= 64 at the layer's
    // shapes (more resident workgroups per CU hide the load latency better than 128x128)
    return run_mfma<1, 4, 4, 2, kEpiStore>(a, st);
  }
  if (a.M <= 32) return run_mfma<1, 4, 2, 1, kEpiOutputGate>(a, st);
  return run_mfma<1, 4, 4, 2, kEpiOutputGate>(a, st);
}

int launch_gate_rowq(const LinearArgs& a, const RowQuant& o, hipStream_t st) {
  TESM_REQUIRE(a.epilogue == kEpiOutputGate, kErrInvalidArg, "gate_rowq: needs the output-gate operands");
  TESM_REQUIRE(a.M >= 0 && a.N >= 1 && a.N <= 1024, kErrUnsupported, "gate_rowq: needs 1 <= d_model <= 1024");
  TESM_REQUIRE(a.Kp >= kKTile && a.Kp % kKTile == 0, kErrInvalidArg, "gate_rowq: Kp must be a multiple of 128");
  TESM_REQUIRE(a.out_dt == kF32 || a.out_dt == kBF16, kErrInvalidArg, "gate_rowq: dtype must be 0 or 1");
  if (a.M == 0) return kOk;
  if (int rc = check_operand(a.op[0], a.Kp, "op0")) return rc;
  if (int rc = check_operand(a.op[1], a.Kp, "op1")) return rc;
  TESM_REQUIRE(a.local && a.gate && a.ld_local >= a.N && a.ld_gate >= a.N, kErrInvalidArg,
               "gate_rowq: need local and gate operands");
  TESM_REQUIRE(o.q && o.s && o.rs && o.ldq >= a.N && o.ldq % 16 == 0 && aligned(o.q, 16), kErrInvalidArg,
               "gate_rowq: bad code outputs");
  TESM_REQUIRE(!o.y || o.ldy >= a.N, kErrInvalidArg, "gate_rowq: bad y output");
  const int64_t nct = (a.N + 63) / 64;
  if (nct <= 1) return run_rowq<1>(a, o, st);
  if (nct <= 2) return run_rowq<2>(a, o, st);
  if (nct <= 3) return run_rowq<3>(a, o, st);
  if (nct <= 4) return run_rowq<4>(a, o, st);
  if (nct <= 6) return run_rowq<6>(a, o, st);
  if (nct <= 8) return run_rowq<8>(a, o, st);
  if (nct <= 12) return run_rowq<12>(a, o, st);
  return run_rowq<16>(a, o, st);
}

}  // namespace tesm
