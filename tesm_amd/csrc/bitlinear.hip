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
#include <cstdlib>

#include "tesm_hip_internal.h"

namespace tesm {

namespace {

__device__ __forceinline__ uint32_t unpack_u(uint32_t w, int s) { return (w >> (2 * s)) & 0x03030303u; }

// ---------------------------------------------------------------------------
// GEMV
// ---------------------------------------------------------------------------
// RPG: output rows per lane group (independent loads in flight per lane).
template <int LPR, int MR, int NCH, int OUT_DT, int RPG = 4>
__global__ __launch_bounds__(256) void gemv_kernel(LinearArgs a) {
  constexpr int GPW = 64 / LPR;   // lane groups per wave
  const LinearOperand& o = a.op[0];
  const int lane = threadIdx.x & 63;
  const int g = lane & (LPR - 1);
  const int64_t group = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * GPW + lane / LPR;
  const int64_t n0 = group * RPG;
  if (n0 >= a.N) return;
  const int64_t nch = a.Kp / 64;

  // the epilogue's operands first, from clamped indices (raw bits, converted where used): requested
  // after the products they would each cost one more memory round trip at the end of the kernel
  float sxv[MR];
  int32_t rsv[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const int64_t mc = m < a.M ? m : a.M - 1;
    sxv[m] = o.s_x[mc];
    rsv[m] = o.rowsum[mc];
  }
  float cwv[RPG];
  uint32_t bias_bits[RPG];
  const void* bias_src = a.bias ? a.bias : static_cast<const void*>(o.c_w);  // a valid address either way
#pragma unroll
  for (int r = 0; r < RPG; ++r) {
    const int64_t nc = n0 + r < a.N ? n0 + r : a.N - 1;
    cwv[r] = o.c_w[o.c_w_per_row ? nc : 0];
    bias_bits[r] = ld_bits<OUT_DT>(bias_src, a.bias ? nc : 0);
  }

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
  // the row scales and sums are wave-uniform (scalar loads): pinned here, while the vector loads above
  // are in flight, so the compiler does not sink them past the products into the storing lanes' branch
#pragma unroll
  for (int m = 0; m < MR; ++m) asm volatile("" : "+s"(sxv[m]), "+s"(rsv[m]));
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
      acc[r][m] = wave_sum_i<LPR>(acc[r][m]);  // DPP / swizzle steps (integer sums: any order is exact)
    }
  // every lane forms the outputs (so the epilogue's loads are waited for here, not after the branch)
  float outv[RPG][MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    const float inv = 1.0f / sxv[m];
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
      acc[r][m] -= rsv[m];
      float v = (static_cast<float>(acc[r][m]) * inv) * cwv[r];
      if (a.bias) v = v + from_bits<OUT_DT>(bias_bits[r]);
      outv[r][m] = v;
    }
  }
  if (g != 0) return;
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= a.M) break;
#pragma unroll
    for (int r = 0; r < RPG; ++r) {
      const int64_t n = n0 + r;
      if (n >= a.N) break;
      if (a.acc_dump) a.acc_dump[m * a.N + n] = acc[r][m];
      st<OUT_DT>(a.out, m * a.ldo + n, outv[r][m]);
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
// Inside an A fragment lane L's 16 bytes sit at slot a_slot(L, ks): the low 4 bits are XORed with
// the code group so that the staging stores (8 lanes per row, one row's 8 code groups) hit
// distinct banks; the 64 lanes of a fragment read still form a permutation of its 64 slots.
__device__ __forceinline__ int a_slot(int lane, int ks) {
  return ((lane & 15) ^ (4 * (lane >> 4)) ^ (2 * ks)) + 16 * (lane >> 4);
}
__device__ __forceinline__ int a_frag_off(int r, int kg) {
  return (((r >> 4) * 2 + (kg >> 2)) << 10) + (a_slot((r & 15) + 16 * (kg & 3), kg >> 2) << 4);
}
// B stays in its global order in LDS: column n of the tile owns 32 bytes (the 128 codes of the K
// tile), its two 16-byte halves swapped on every other group of 8 columns so that a fragment read
// (16 columns x 4 dwords) covers 64 distinct banks.
__device__ __forceinline__ int b_col_off(int n, int half) { return n * 32 + 16 * (half ^ ((n >> 3) & 1)); }

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

template <class C>
__device__ __forceinline__ void gemm_sstore(const int (&la)[C::A_PT], const int (&lb)[C::B_PT],
                                            const bool (&vb)[C::B_PT], const v4i (&ra)[C::A_PT],
                                            const v4i (&rb)[C::B_PT], char* stage) {
#pragma unroll
  for (int p = 0; p < C::A_PT; ++p) *reinterpret_cast<v4i*>(stage + la[p]) = ra[p];
#pragma unroll
  for (int p = 0; p < C::B_PT; ++p)
    if (vb[p]) *reinterpret_cast<v4i*>(stage + lb[p]) = rb[p];
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
    lb[p] = C::A_BYTES + b_col_off(c >> 1, c & 1);
  }
  const int64_t nk = Kp / C::BK;
  const int aoff0 = a_slot(lane, 0) * 16, aoff1 = a_slot(lane, 1) * 16;
  // one 128-deep K tile from an LDS stage
  auto compute = [&](const char* cur) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v4i af[TM];
      uint32_t bw[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const v4i*>(cur + (((wm * TM + i) * 2 + ks) << 10) + (ks ? aoff1 : aoff0));
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bw[j] = *reinterpret_cast<const uint32_t*>(cur + C::A_BYTES + b_col_off((wn * TN + j) * 16 + (lane & 15), ks) +
                                                   4 * (lane >> 4));
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const v4i bf = unpack_frag(bw[j]);
        // weights as the MFMA's A operand: the accumulator comes out transposed, so each lane holds
        // 4 consecutive output columns of one row (vector stores in the epilogue)
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, af[i], acc[i][j], 0, 0, 0);
      }
    }
  };
  // Two register sets keep two K tiles of global loads in flight beyond the one in LDS: set 0
  // holds even tiles, set 1 odd tiles; loads past the last tile re-read it (never computed).
  v4i ra0[C::A_PT], rb0[C::B_PT], ra1[C::A_PT], rb1[C::B_PT];
  auto kofs = [&](int64_t kt) { return (kt < nk ? kt : nk - 1) * C::BK; };
  char* const s0 = smem;
  char* const s1 = smem + C::STAGE;
  gemm_gload<C>(pa, pb, vb, kofs(0), ra0, rb0);
  gemm_gload<C>(pa, pb, vb, kofs(1), ra1, rb1);
  gemm_sstore<C>(la, lb, vb, ra0, rb0, s0);
  __syncthreads();
  gemm_gload<C>(pa, pb, vb, kofs(2), ra0, rb0);
  int64_t kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    compute(s0);                                     // tile kt
    gemm_sstore<C>(la, lb, vb, ra1, rb1, s1);        // tile kt + 1
    __syncthreads();
    gemm_gload<C>(pa, pb, vb, kofs(kt + 3), ra1, rb1);
    compute(s1);                                     // tile kt + 1
    gemm_sstore<C>(la, lb, vb, ra0, rb0, s0);        // tile kt + 2 (past the end: never computed)
    __syncthreads();
    gemm_gload<C>(pa, pb, vb, kofs(kt + 4), ra0, rb0);
  }
  if (kt < nk) compute(s0);                          // odd number of K tiles
  __syncthreads();  // the stages may be refilled by a following main loop (output-gate products)
}

// Tile order for a 1-D grid: workgroups are handed to the 8 XCDs round-robin by id, so id is
// mapped to a tile such that each XCD gets a contiguous run of tiles (row-major over
// (M tile, N tile)); consecutive tiles of one XCD share A rows in that XCD's L2.
__device__ __forceinline__ void xcd_tile_of(int64_t pid, int64_t ntm, int64_t ntn, int64_t& tm, int64_t& tn) {
  constexpr int64_t kXcd = 8;
  const int64_t total = ntm * ntn;
  const int64_t x = pid % kXcd, i = pid / kXcd;
  const int64_t q = total / kXcd, r = total % kXcd;
  const int64_t tile = x * q + (x < r ? x : r) + i;
  // groups of kGroupM M-tile rows with M fastest: the tiles an XCD runs at once cover a few M rows
  // and N columns, so both operands' K slabs are shared through its L2
  constexpr int64_t kGroupM = 8;
  const int64_t g = tile / (kGroupM * ntn);
  const int64_t first_m = g * kGroupM;
  const int64_t gsz = ntm - first_m < kGroupM ? ntm - first_m : kGroupM;
  const int64_t local = tile - g * kGroupM * ntn;
  tm = first_m + local % gsz;
  tn = local / gsz;
}
__device__ __forceinline__ void xcd_tile(int64_t ntm, int64_t ntn, int64_t& tm, int64_t& tn) {
  xcd_tile_of(blockIdx.x, ntm, ntn, tm, tn);
}

// With the weights as the A operand, element r of lane L's accumulator is output row L%16 and
// output column 4*(L/16) + r of the 16 x 16 tile.
template <int OUT_DT>
__device__ __forceinline__ void store4(void* out, int64_t idx, const float (&v)[4], bool vec) {
  if (vec) {
    if constexpr (OUT_DT == kBF16) {
      const uint32_t lo = pack_bf16x2(v[0], v[1]);
      const uint32_t hi = pack_bf16x2(v[2], v[3]);
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

// Two-product epilogues on the rounded products p0 = rnd(v0), p1 = rnd(v1):
//   output gate  y = rnd(rnd(local + rnd(sigmoid(gate) * p0)) + p1)      (tesm.py:1256-1261)
//   SwiGLU       h = rnd(rnd(silu(p0)) * p1), silu(x) = x * sigmoid(x)  (mixer_seq_simple.py:63-64)
template <int EPI, int OUT_DT>
__device__ __forceinline__ float dual_epi(float p0, float p1, float local, float gate) {
  if constexpr (EPI == kEpiOutputGate) {
    const float g = rnd<OUT_DT>(sigmoidf_(gate));
    return rnd<OUT_DT>(rnd<OUT_DT>(local + rnd<OUT_DT>(g * p0)) + p1);
  } else {
    return rnd<OUT_DT>(rnd<OUT_DT>(p0 * sigmoidf_(p0)) * p1);
  }
}

// kEpiGates: the region of the 32-column tile that starts at column n (0: stored as is, 1: tanh,
// 2: biased sigmoid, 3: sigmoid).  act_n0 and act_w are multiples of 32, so a tile lies in one region
// and the region is uniform over the wave.
__device__ __forceinline__ int gate_region(const LinearArgs& a, int64_t n) {
  const int64_t r = n - a.act_n0;
  return r < 0 ? 0 : r < a.act_w ? 1 : r < 2 * a.act_w ? 2 : r < 3 * a.act_w ? 3 : 0;
}

// The MIMO gates on four consecutive columns n .. n + 3 of one region (tesm_mimo.py:958-961), each
// on the product rounded to the output dtype: the float ops a scan would apply to the stored
// products, so the values it reads are the ones it would have computed.
template <int DT>
__device__ __forceinline__ void gate_act4(const LinearArgs& a, int kind, int64_t n, float (&v)[4]) {
  if (kind == 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = rnd<DT>(tanhf_(rnd<DT>(v[r])));
  } else if (kind == 2) {
    const int64_t c = n - a.act_n0 - a.act_w;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = rnd<DT>(sigmoidf_(rnd<DT>(rnd<DT>(v[r]) + ld<DT>(a.act_bias, c + r))));
  } else if (kind == 3) {
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = rnd<DT>(sigmoidf_(rnd<DT>(v[r])));
  }
}

// General epilogue of the 16 x 16 tiles of one wave (tile rows wm*TM.., columns wn*TN..): scale the
// exact accumulators, optional bias / accumulator dump, or the output gate
// y = local + sigmoid(gate) * state_proj + ent_proj in the module dtype's op order.
// Operands of one 16·TM × 16·TN epilogue tile (activation scales and code sums, weight scales, bias,
// output-gate inputs) for the split-K kernels, read in straight-line code with rows and columns clamped into range (values
// at clamped positions are never stored), so they are all in flight together and can be issued
// before the K loop.
template <int TM, int TN, int EPI, int OUT_DT>
struct Epi16In {
  float sx0[TM], sx1[TM];  // activation scales and code sums of the lane's rows
  int32_t rs0[TM], rs1[TM];
  float cw0[TN][4], cw1[TN][4];
  uint32_t bias[TN][4];
  uint32_t lo[TM][TN][4], gt[TM][TN][4];
};

template <int TM, int TN, int EPI, int OUT_DT>
__device__ __forceinline__ void epi16_load(const LinearArgs& a, Epi16In<TM, TN, EPI, OUT_DT>& e, int64_t m0,
                                           int64_t n0, int lane) {
  const LinearOperand& o0 = a.op[0];
  const LinearOperand& o1 = a.op[1];
  const void* bias = a.bias ? a.bias : static_cast<const void*>(o0.c_w);  // no bias: a valid dummy address
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t nb = n0 + j * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = nb + r < a.N ? nb + r : a.N - 1;
      e.cw0[j][r] = o0.c_w[o0.c_w_per_row ? n : 0];
      if constexpr (epi_dual(EPI)) e.cw1[j][r] = o1.c_w[o1.c_w_per_row ? n : 0];
      if constexpr (EPI == kEpiStore) e.bias[j][r] = ld_bits<OUT_DT>(bias, a.bias ? n : 0);
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + i * 16 + (lane & 15), mc = m < a.M ? m : a.M - 1;
    e.sx0[i] = o0.s_x[mc];
    e.rs0[i] = o0.rowsum[mc];
    if constexpr (epi_dual(EPI)) {
      e.sx1[i] = o1.s_x[mc];
      e.rs1[i] = o1.rowsum[mc];
    }
  }
  if constexpr (EPI == kEpiOutputGate) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = m0 + i * 16 + (lane & 15), mc = m < a.M ? m : a.M - 1;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t nb = n0 + j * 16 + 4 * (lane >> 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t n = nb + r < a.N ? nb + r : a.N - 1;
          e.lo[i][j][r] = ld_bits<OUT_DT>(a.local, mc * a.ld_local + n);
          e.gt[i][j][r] = ld_bits<OUT_DT>(a.gate, mc * a.ld_gate + n);
        }
      }
    }
  }
}

// The split-K kernels' epilogue (one wave owns the whole tile) on operands read by epi16_load.
template <int TM, int TN, int EPI, int OUT_DT>
__device__ __forceinline__ void epilogue16_pre(const LinearArgs& a, const v4i (&acc0)[TM][TN],
                                               const v4i (&acc1)[TM][TN], const Epi16In<TM, TN, EPI, OUT_DT>& e,
                                               int64_t m0, int64_t n0, int lane) {
  const bool vout = vec4_ok<OUT_DT>(a.out, a.ldo);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + i * 16 + (lane & 15);
    if (m >= a.M) continue;
    const float inv0 = 1.0f / e.sx0[i];
    const int32_t rs0 = e.rs0[i];
    float inv1 = 0.0f;
    int32_t rs1 = 0;
    if constexpr (epi_dual(EPI)) {
      inv1 = 1.0f / e.sx1[i];
      rs1 = e.rs1[i];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t nb = n0 + j * 16 + 4 * (lane >> 4);
      if (nb >= a.N) continue;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t n = nb + r;
        const int32_t a0 = acc0[i][j][r] - rs0;
        if (a.acc_dump && n < a.N) a.acc_dump[m * a.N + n] = a0;
        const float v0 = (static_cast<float>(a0) * inv0) * e.cw0[j][r];
        if constexpr (EPI == kEpiStore) {
          v[r] = a.bias ? v0 + from_bits<OUT_DT>(e.bias[j][r]) : v0;
        } else {
          const float v1 = rnd<OUT_DT>((static_cast<float>(acc1[i][j][r] - rs1) * inv1) * e.cw1[j][r]);
          if constexpr (EPI == kEpiOutputGate)
            v[r] = dual_epi<EPI, OUT_DT>(rnd<OUT_DT>(v0), v1, from_bits<OUT_DT>(e.lo[i][j][r]),
                                         from_bits<OUT_DT>(e.gt[i][j][r]));
          else
            v[r] = dual_epi<EPI, OUT_DT>(rnd<OUT_DT>(v0), v1, 0.0f, 0.0f);
        }
      }
      if (nb + 3 < a.N) {
        store4<OUT_DT>(a.out, m * a.ldo + nb, v, vout);
      } else {
        for (int r = 0; r < 4 && nb + r < a.N; ++r) st<OUT_DT>(a.out, m * a.ldo + nb + r, v[r]);
      }
    }
  }
}

template <int TM, int TN, int EPI, int OUT_DT>
__device__ __forceinline__ void epilogue16(const LinearArgs& a, const v4i (&acc0)[TM][TN], const v4i (&acc1)[TM][TN],
                                           int64_t m0, int64_t n0, int wm, int wn, int lane) {
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
    if constexpr (epi_dual(EPI)) {
      inv1 = 1.0f / o1.s_x[m];
      rs1 = o1.rowsum[m];
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t nb = n0 + (wn * TN + j) * 16 + 4 * (lane >> 4);
      if (nb >= a.N) continue;
      const bool full = nb + 3 < a.N;
      float v[4], lo[4] = {0.0f, 0.0f, 0.0f, 0.0f}, gt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
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
          const float v1 = rnd<OUT_DT>((static_cast<float>(acc1[i][j][r] - rs1) * inv1) * cw1);
          v[r] = dual_epi<EPI, OUT_DT>(rnd<OUT_DT>(v0), v1, lo[r], gt[r]);
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
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w / WN, wn = w % WN;
  const LinearOperand& o0 = a.op[0];
  // plain products (one scalar c_w, no bias, no accumulator dump) take the short epilogue, whose
  // per-row operands are requested before the main loop
  const bool plain = EPI == kEpiStore && !o0.c_w_per_row && !a.bias && !a.acc_dump;
  float sx[TM];
  int32_t rsum[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + (wm * TM + i) * 16 + (lane & 15);
    const int64_t mc = m < a.M ? m : a.M - 1;
    sx[i] = o0.s_x[mc];
    rsum[i] = o0.rowsum[mc];
  }
  const float cws = o0.c_w[0];
  mfma_mainloop<C, WN, TM, TN>(a.op[0], a.M, a.N, m0, n0, a.Kp, acc0, smem);
  if constexpr (epi_dual(EPI)) mfma_mainloop<C, WN, TM, TN>(a.op[1], a.M, a.N, m0, n0, a.Kp, acc1, smem);

  if (plain) {
    const int nrem = static_cast<int>(std::min<int64_t>(a.N - n0, C::BN));  // columns of this tile
    const bool vout = vec4_ok<OUT_DT>(a.out, a.ldo);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = m0 + (wm * TM + i) * 16 + (lane & 15);
      if (m >= a.M) continue;
      const float inv = 1.0f / sx[i];
      char* orow = static_cast<char*>(a.out) + (m * a.ldo + n0) * (OUT_DT == kBF16 ? 2 : 4);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int nb = (wn * TN + j) * 16 + 4 * (lane >> 4);  // within the tile
        if (nb >= nrem) continue;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = (static_cast<float>(acc0[i][j][r] - rsum[i]) * inv) * cws;
        if (vout && nb + 4 <= nrem) {
          store4<OUT_DT>(orow, nb, v, true);
        } else {
          for (int r = 0; r < 4 && nb + r < nrem; ++r) st<OUT_DT>(orow, nb + r, v[r]);
        }
      }
    }
    return;
  }
  epilogue16<TM, TN, EPI, OUT_DT>(a, acc0, acc1, m0, n0, wm, wn, lane);
}

// ---------------------------------------------------------------------------
// Small-M products (decode batches, M <= 16*TM): one workgroup per 16*TM x 16*TN output tile, the K
// loop split over its NW waves.  Wave w takes the 256-code blocks w, w + NW, ...; per block, lane L
// (weight column / activation row L%16, group g = L/16) reads one b128 of packed weights per column
// tile (codes 64g .. 64g+63 of the block) and four b128 of activation codes per row tile (the same
// 64 codes of its row).  In k-step s the lane feeds codes 64g + 16s .. +15 to both MFMA operands, so
// every code of the block meets its weight exactly once.  Operands come straight from global
// memory with the next block's loads issued before the current block's MFMAs; the waves' int32
// partial sums are added through LDS (exact, order-free) and wave 0 runs the epilogue.  This gives
// N/(16*TN) workgroups of NW waves instead of the LDS-staged kernel's N/64 single-stream tiles.
template <int TM, int TN>
struct SkinnyRegs {
  uint4 w[TN];      // packed weights of the block: dword s feeds k-step s
  v4i x[TM][4];     // activation codes: x[i][s] feeds k-step s of row tile i
};

template <int TM, int TN>
__device__ __forceinline__ void skinny_load(SkinnyRegs<TM, TN>& r, const uint8_t* const (&pw)[TN],
                                            const int8_t* const (&pa)[TM], int64_t kb, bool live) {
  if (live) {
#pragma unroll
    for (int j = 0; j < TN; ++j) r.w[j] = *reinterpret_cast<const uint4*>(pw[j] + 64 * kb);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int s = 0; s < 4; ++s) r.x[i][s] = *reinterpret_cast<const v4i*>(pa[i] + 256 * kb + 16 * s);
  } else {  // codes past Kp: zero activations contribute nothing whatever the weights
#pragma unroll
    for (int j = 0; j < TN; ++j) r.w[j] = make_uint4(0x55555555u, 0x55555555u, 0x55555555u, 0x55555555u);
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int s = 0; s < 4; ++s) r.x[i][s] = v4i{0, 0, 0, 0};
  }
}

template <int TM, int TN>
__device__ __forceinline__ void skinny_mma(const SkinnyRegs<TM, TN>& r, v4i (&acc)[TM][TN]) {
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint32_t wd = s == 0 ? r.w[j].x : s == 1 ? r.w[j].y : s == 2 ? r.w[j].z : r.w[j].w;
      const v4i bf = unpack_frag(wd);
#pragma unroll
      for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bf, r.x[i][s], acc[i][j], 0, 0, 0);
    }
}

// K loop of one wave over the blocks w, w + NW, ... of Kp (a trailing 128-code half block is read by
// groups 0 and 1 only).
template <int NW, int TM, int TN>
__device__ __forceinline__ void skinny_loop(const LinearOperand& o, int64_t M, int64_t N, int64_t m0, int64_t n0,
                                            int64_t Kp, int w, int lane, v4i (&acc)[TM][TN]) {
  const int g = lane >> 4, l16 = lane & 15;
  const uint8_t* pw[TN];
  const int8_t* pa[TM];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = n0 + 16 * j + l16;
    pw[j] = o.w + (n < N ? n : N - 1) * o.ldw + 16 * g;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + 16 * i + l16;
    pa[i] = o.q + (m < M ? m : M - 1) * o.ldq + 64 * g;
  }
  const int64_t nblk = (Kp + 255) / 256;
  const bool half_tail = (Kp & 255) != 0;  // last block holds 128 codes: groups 0 and 1
  auto live = [&](int64_t kb) { return kb < nblk && (!half_tail || kb + 1 < nblk || g < 2); };
  SkinnyRegs<TM, TN> r0, r1;
  int64_t kb = w;
  skinny_load<TM, TN>(r0, pw, pa, kb, live(kb));
  for (; kb < nblk; kb += 2 * NW) {
    skinny_load<TM, TN>(r1, pw, pa, kb + NW, live(kb + NW));
    skinny_mma<TM, TN>(r0, acc);
    if (kb + NW >= nblk) break;
    skinny_load<TM, TN>(r0, pw, pa, kb + 2 * NW, live(kb + 2 * NW));
    skinny_mma<TM, TN>(r1, acc);
  }
}

template <int NW, int TM, int TN, int EPI, int OUT_DT>
__device__ __forceinline__ void skinny_body(const LinearArgs& a, int64_t m0, int64_t n0) {
  constexpr int NOP = epi_dual(EPI) ? 2 : 1;
  __shared__ v4i red[(NW - 1) * NOP * TM * TN * 64];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  Epi16In<TM, TN, EPI, OUT_DT> ein;  // wave 0's epilogue operands, in flight during the K loop
  if (w == 0) epi16_load<TM, TN, EPI, OUT_DT>(a, ein, m0, n0, lane);
  v4i acc0[TM][TN], acc1[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      acc0[i][j] = v4i{0, 0, 0, 0};
      acc1[i][j] = v4i{0, 0, 0, 0};
    }
  skinny_loop<NW, TM, TN>(a.op[0], a.M, a.N, m0, n0, a.Kp, w, lane, acc0);
  if constexpr (epi_dual(EPI)) skinny_loop<NW, TM, TN>(a.op[1], a.M, a.N, m0, n0, a.Kp, w, lane, acc1);
  const int nblk = static_cast<int>((a.Kp + 255) / 256), nact = nblk < NW ? nblk : NW;  // waves with blocks
  if (w > 0 && w < nact) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        red[((((w - 1) * NOP) * TM + i) * TN + j) * 64 + lane] = acc0[i][j];
        if constexpr (NOP == 2) red[((((w - 1) * NOP + 1) * TM + i) * TN + j) * 64 + lane] = acc1[i][j];
      }
  }
  __syncthreads();
  if (w != 0) return;
  for (int src = 0; src < nact - 1; ++src)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        acc0[i][j] += red[(((src * NOP) * TM + i) * TN + j) * 64 + lane];
        if constexpr (NOP == 2) acc1[i][j] += red[(((src * NOP + 1) * TM + i) * TN + j) * 64 + lane];
      }
  epilogue16_pre<TM, TN, EPI, OUT_DT>(a, acc0, acc1, ein, m0, n0, lane);
}

template <int NW, int TM, int TN, int EPI, int OUT_DT>
__global__ __launch_bounds__(NW * 64) void skinny_kernel(LinearArgs a) {
  const int64_t ntn = (a.N + 16 * TN - 1) / (16 * TN);
  const int64_t tm = blockIdx.x / ntn, tn = blockIdx.x - tm * ntn;
  skinny_body<NW, TM, TN, EPI, OUT_DT>(a, tm * 16 * TM, tn * 16 * TN);
}

// The same product with the activation quantization fused (decode-size batches): the workgroup
// quantizes its 16 TM rows of x into LDS exactly as quant_act_kernel does (absmax scale per row,
// int8 codes in layout 1, code sums), then runs the split-K body on them.  Every workgroup of a row
// tile repeats the quantization (a few KB of L2 reads each) in exchange for one launch fewer.  LDS
// rows are Kp + 16 bytes apart, so the 16 rows a K-step reads fall on distinct banks.
// G > 0: a lane's at most G groups stay in registers between the amax and the code pass (one read
// of the row, all loads issued before the first use; needs VEC rows with K % 16 == 0); G == 0: the
// row is read twice.
template <int NW, int TM, int TN, int OUT_DT, int DT, bool VEC, int G>
__global__ __launch_bounds__(NW * 64) void skinny_fq_kernel(LinearArgs a, FusedQuantIn f) {
  extern __shared__ __attribute__((aligned(16))) char lds_fq[];
  constexpr int R = 16 * TM, LPR = NW * 64 / R;  // rows of the tile, lanes per row
  const int64_t ntn = (a.N + 16 * TN - 1) / (16 * TN);
  const int64_t tm = blockIdx.x / ntn, tn = blockIdx.x - tm * ntn;
  const int64_t m0 = tm * 16 * TM, n0 = tn * 16 * TN;
  const int64_t lstride = a.Kp + 16;
  int8_t* codes = reinterpret_cast<int8_t*>(lds_fq);
  float* sc_l = reinterpret_cast<float*>(lds_fq + R * lstride);
  int32_t* rs_l = reinterpret_cast<int32_t*>(sc_l + R);
  {
    const int r = threadIdx.x / LPR, g0 = threadIdx.x % LPR;  // LPR consecutive lanes per row
    const int64_t m = m0 + r, ngroups = a.Kp / 16;
    int8_t* crow = codes + r * lstride;
    if (G > 0) {
      // Straight-line code: the lane's G groups are loaded (16-byte loads, all issued before the first
      // use) from row min(m, M - 1), groups past K re-reading the row's last group; both are zeroed
      // or discarded below.  Needs 16-byte aligned rows and K % 16 == 0.
      const int64_t mc = m < a.M ? m : a.M - 1;
      float v[G > 0 ? G : 1][16];
      load_groups<DT, (G > 0 ? G : 1), LPR>(f.x, mc * f.ldx, f.K, g0, v);
      float amax = 0.0f;
#pragma unroll
      for (int gi = 0; gi < G; ++gi)
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[gi][i]));
      amax = wave_max<LPR>(amax);
      const bool live = m < a.M;  // rows past M: zero codes, scale 1, sum 0
      const float sc = act_scale<DT>(amax, f.eps);
      int32_t rs = 0;
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        const int64_t g = g0 + LPR * gi;
        const uint4 c = group_codes<DT>(v[gi], sc, 1, rs);
        if (g < ngroups) *reinterpret_cast<uint4*>(crow + 16 * g) = live ? c : make_uint4(0, 0, 0, 0);
      }
      rs = wave_sum_i<LPR>(rs);
      if (g0 == 0) {
        sc_l[r] = live ? sc : 1.0f;
        rs_l[r] = live ? rs : 0;
      }
    } else if (m < a.M) {
      const int64_t base = m * f.ldx;
      float amax = 0.0f;
      for (int64_t g = g0; g < ngroups; g += LPR) {
        float v[16];
        load_group<DT, VEC>(f.x, base, f.K, g, v);
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
      }
      amax = wave_max<LPR>(amax);
      const float sc = act_scale<DT>(amax, f.eps);
      int32_t rs = 0;
      for (int64_t g = g0; g < ngroups; g += LPR) {
        float v[16];
        load_group<DT, VEC>(f.x, base, f.K, g, v);
        *reinterpret_cast<uint4*>(crow + 16 * g) = group_codes<DT>(v, sc, 1, rs);
      }
      rs = wave_sum_i<LPR>(rs);
      if (g0 == 0) {
        sc_l[r] = sc;
        rs_l[r] = rs;
      }
    } else {  // rows past M: zero codes (never stored)
      for (int64_t g = g0; g < ngroups; g += LPR) *reinterpret_cast<uint4*>(crow + 16 * g) = make_uint4(0, 0, 0, 0);
      if (g0 == 0) {
        sc_l[r] = 1.0f;
        rs_l[r] = 0;
      }
    }
  }
  __syncthreads();
  LinearArgs b = a;  // operand 0 now reads the LDS copy, indexed by global row as before
  b.op[0].q = codes - m0 * lstride;
  b.op[0].ldq = lstride;
  b.op[0].s_x = sc_l - m0;
  b.op[0].rowsum = rs_l - m0;
  skinny_body<NW, TM, TN, kEpiStore, OUT_DT>(b, m0, n0);
}

// ---------------------------------------------------------------------------
// GEMM on v_mfma_i32_32x32x32_i8, which on gfx950 delivers about twice the int8 rate of the
// 16x16x64 form.  Block tile BM x BN (waves WM x WN, each TM x TN tiles of 32 x 32), K tiles of
// 128 codes = 8 chunks of 16 codes in 4 k-steps.  Weights are the MFMA's A operand: in k-step s,
// lane L feeds weight column L%32 with chunk 4*(L/32) + s (one packed dword, unpacked in registers)
// and activation row L%32 with the same chunk (16 bytes); any pairing of chunks to k-steps gives the
// same sums as long as both operands use it, and this one makes a lane's four weight dwords of a K
// tile one contiguous 16-byte read.  Accumulator element r of lane L is weight column
// 8*(r/4) + 4*(L/32) + r%4 and activation row L%32, so every lane stores runs of 4 consecutive
// outputs.
//
// LDS, per stage (bank model measured on the device: 16-byte reads are served 16 lanes per pass over
// 256 bytes, 16-byte writes 8 lanes per pass over 128 bytes): activations in chunk planes
// [q][row][16 bytes] with row slot row ^ q, so a fragment read (16 consecutive rows, one chunk) and
// a staging store (8 chunks of one row) both hit distinct banks; packed weights [col][half][16 bytes]
// with the halves swapped on odd groups of 8 columns, so a fragment read (16 columns, one half)
// covers all banks and a staging store (4 columns x 2 halves) 128 contiguous bytes.
typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <int WM, int WN, int TM, int TN>
struct Cfg32 {
  static constexpr int NT = WM * WN * 64;
  static constexpr int BM = WM * TM * 32, BN = WN * TN * 32, BK = 128;
  static constexpr int A_BYTES = BM * BK;
  static constexpr int B_BYTES = BN * BK / 4;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_CHUNKS = BM * BK / 16;
  static constexpr int B_CHUNKS = BN * BK / 64;
  static constexpr int A_PT = (A_CHUNKS + NT - 1) / NT;
  static constexpr int B_PT = (B_CHUNKS + NT - 1) / NT;
};

template <int BM>
__device__ __forceinline__ int a32_off(int row, int q) { return q * BM * 16 + (row ^ q) * 16; }
__device__ __forceinline__ int b32_off(int col, int h) { return col * 32 + 16 * (h ^ ((col >> 3) & 1)); }

template <class C, int WN, int TM, int TN>
__device__ __forceinline__ void mfma32_mainloop(const LinearOperand& o, int64_t M, int64_t N, int64_t m0, int64_t n0,
                                                int64_t Kp, v16i (&acc)[TM][TN], char* smem) {
  const int t = threadIdx.x;
  __builtin_assume(t < C::NT);
  const int lane = t & 63, w = t >> 6;
  const int wm = w / WN, wn = w % WN;
  constexpr bool kAllA = (C::A_CHUNKS % C::NT) == 0;
  constexpr bool kAllB = (C::B_CHUNKS % C::NT) == 0;
  static_assert(kAllA, "A chunks must divide evenly over the workgroup");

  // rows past M / columns past N read the last valid one and only feed outputs never stored
  const int8_t* pa[C::A_PT];
  int la[C::A_PT];
#pragma unroll
  for (int p = 0; p < C::A_PT; ++p) {
    const int c = t + p * C::NT;
    const int64_t m = m0 + (c >> 3);
    pa[p] = o.q + (m < M ? m : M - 1) * o.ldq + 16 * (c & 7);
    la[p] = a32_off<C::BM>(c >> 3, c & 7);
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
    lb[p] = C::A_BYTES + b32_off(c >> 1, c & 1);
  }
  const int64_t nk = Kp / C::BK;
  auto gload = [&](int64_t kt, v4i (&ra)[C::A_PT], v4i (&rb)[C::B_PT]) {
    const int64_t k0 = (kt < nk ? kt : nk - 1) * C::BK;
#pragma unroll
    for (int p = 0; p < C::A_PT; ++p) ra[p] = *reinterpret_cast<const v4i*>(pa[p] + k0);
#pragma unroll
    for (int p = 0; p < C::B_PT; ++p)
      if (vb[p]) rb[p] = *reinterpret_cast<const v4i*>(pb[p] + k0 / 4);
  };
  auto sstore = [&](const v4i (&ra)[C::A_PT], const v4i (&rb)[C::B_PT], char* stage) {
#pragma unroll
    for (int p = 0; p < C::A_PT; ++p) *reinterpret_cast<v4i*>(stage + la[p]) = ra[p];
#pragma unroll
    for (int p = 0; p < C::B_PT; ++p)
      if (vb[p]) *reinterpret_cast<v4i*>(stage + lb[p]) = rb[p];
  };
  // per-lane fragment offsets: chunk 4*(lane/32) + s of the lane's row / column
  const int hq = 4 * (lane >> 5);
  int ar[4][TM];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int i = 0; i < TM; ++i) ar[s][i] = a32_off<C::BM>((wm * TM + i) * 32 + (lane & 31), hq + s);
  int br[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) br[j] = C::A_BYTES + b32_off((wn * TN + j) * 32 + (lane & 31), lane >> 5);
  auto compute = [&](const char* cur) {
    v4i bw[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) bw[j] = *reinterpret_cast<const v4i*>(cur + br[j]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      v4i af[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const v4i*>(cur + ar[s][i]);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const v4i bf = unpack_frag(static_cast<uint32_t>(bw[j][s]));
#pragma unroll
        for (int i = 0; i < TM; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[i], acc[i][j], 0, 0, 0);
      }
    }
  };
  // two register sets keep two K tiles of loads in flight beyond the one in LDS
  v4i ra0[C::A_PT], rb0[C::B_PT], ra1[C::A_PT], rb1[C::B_PT];
  char* const s0 = smem;
  char* const s1 = smem + C::STAGE;
  gload(0, ra0, rb0);
  gload(1, ra1, rb1);
  sstore(ra0, rb0, s0);
  __syncthreads();
  gload(2, ra0, rb0);
  int64_t kt = 0;
  for (; kt + 2 <= nk; kt += 2) {
    compute(s0);
    sstore(ra1, rb1, s1);
    __syncthreads();
    gload(kt + 3, ra1, rb1);
    compute(s1);
    sstore(ra0, rb0, s0);
    __syncthreads();
    gload(kt + 4, ra0, rb0);
  }
  if (kt < nk) compute(s0);
  __syncthreads();
}

// Main loop with direct-to-LDS loads (global_load_lds_dwordx4): NS stages in LDS, no staging
// registers.  One such instruction moves 64 lanes x 16 bytes into 1 KB of LDS in lane order, so the
// layouts are chosen through the lanes' global addresses: activation rows in blocks of 8 rows x 8
// chunks (a row's 8 lanes read one 128-byte line, chunk q of row r lands in slot
// r*8 + (q ^ ((r/2) % 8))), weights in blocks of 32 columns x 2 halves (half h of column n in slot
// 2n + (h ^ ((n/8) % 2))); both make the fragment reads (16 lanes: consecutive rows or columns, one
// chunk) hit 16 distinct 16-byte slots of 256 bytes.  Each wave issues D of these per K tile (with two
// stages the last blocks may leave some waves one short); the wait for tile kt is "at most (NS - 2) *
// D outstanding" (loads past the last K tile re-read it, so the count never shrinks), then one
// barrier, then the refill of the stage the previous tile used.
template <int BM>
__device__ __forceinline__ int a32d_off(int row, int q) { return 16 * (row * 8 + (q ^ ((row >> 1) & 7))); }
__device__ __forceinline__ int b32d_off(int col, int h) { return 16 * (col * 2 + (h ^ ((col >> 3) & 1))); }

__device__ __forceinline__ void lds_dma16(const void* src, char* dst) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst), 16, 0, 0);
}

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt bits [3:0] and
// [15:14], expcnt [6:4] and lgkmcnt [11:8] left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <class C, int WN, int TM, int TN, int NS>
__device__ __forceinline__ void mfma32d_mainloop(const LinearOperand& o, int64_t M, int64_t N, int64_t m0, int64_t n0,
                                                 int64_t Kp, v16i (&acc)[TM][TN], char* smem) {
  constexpr int NW = C::NT / 64;
  constexpr int NA = C::BM / 8, NB = C::BN / 32;  // 1 KB blocks per K tile
  // deeper pipelines count each wave's loads in flight, so they need the same number per wave; two
  // stages wait for all of a wave's loads, so the last blocks may leave some waves one short
  static_assert(NS == 2 || (NA + NB) % NW == 0, "DMA blocks must divide evenly over the waves");
  constexpr int D = (NA + NB + NW - 1) / NW;
  static_assert((NS - 2) * D < 64, "too many loads in flight for vmcnt");
  const int t = threadIdx.x;
  __builtin_assume(t < C::NT);
  const int lane = t & 63, w = t >> 6;
  const int wm = w / WN, wn = w % WN;
  // this lane's source of each of the wave's D blocks (rows / columns past M / N read the last one)
  const char* src[D];
  int dst[D], adv[D];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    const int blk = w + i * NW < NA + NB ? w + i * NW : NA + NB - 1;  // (blocks past the end are never issued)
    if (blk < NA) {
      const int row = blk * 8 + (lane >> 3);
      const int q = (lane & 7) ^ ((row >> 1) & 7);
      const int64_t m = m0 + row;
      src[i] = reinterpret_cast<const char*>(o.q) + (m < M ? m : M - 1) * o.ldq + 16 * q;
      dst[i] = blk * 1024;
      adv[i] = C::BK;
    } else {
      const int col = (blk - NA) * 32 + (lane >> 1);
      const int h = (lane & 1) ^ ((col >> 3) & 1);
      const int64_t n = n0 + col;
      src[i] = reinterpret_cast<const char*>(o.w) + (n < N ? n : N - 1) * o.ldw + 16 * h;
      dst[i] = C::A_BYTES + (blk - NA) * 1024;
      adv[i] = C::BK / 4;
    }
  }
  const int64_t nk = Kp / C::BK;
  auto issue = [&](int64_t kt) {
    const int64_t k = kt < nk ? kt : nk - 1;
    char* stage = smem + static_cast<int>(kt % NS) * C::STAGE;
#pragma unroll
    for (int i = 0; i < D; ++i)
      if ((NA + NB) % NW == 0 || __builtin_amdgcn_readfirstlane(w) + i * NW < NA + NB)  // wave-uniform
        lds_dma16(src[i] + k * adv[i], stage + dst[i]);
  };
  const int hq = 4 * (lane >> 5);
  int ar[4][TM], br[TN];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int i = 0; i < TM; ++i) ar[s][i] = a32d_off<C::BM>((wm * TM + i) * 32 + (lane & 31), hq + s);
#pragma unroll
  for (int j = 0; j < TN; ++j) br[j] = C::A_BYTES + b32d_off((wn * TN + j) * 32 + (lane & 31), lane >> 5);
  // fragments double-buffered by one k-step: the reads for step s + 1 are issued before the MFMAs
  // of step s (scheduling barriers keep the compiler from sinking them), so their latency hides
  // behind TM x TN MFMAs instead of one
  auto compute = [&](const char* cur) {
    v4i bw[TN], af[2][TM];
#pragma unroll
    for (int j = 0; j < TN; ++j) bw[j] = *reinterpret_cast<const v4i*>(cur + br[j]);
#pragma unroll
    for (int i = 0; i < TM; ++i) af[0][i] = *reinterpret_cast<const v4i*>(cur + ar[0][i]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s < 3) {
#pragma unroll
        for (int i = 0; i < TM; ++i) af[(s + 1) & 1][i] = *reinterpret_cast<const v4i*>(cur + ar[s + 1][i]);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const v4i bf = unpack_frag(static_cast<uint32_t>(bw[j][s]));
#pragma unroll
        for (int i = 0; i < TM; ++i)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf, af[s & 1][i], acc[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  __syncthreads();  // the stages may still be read by a previous main loop or epilogue
#pragma unroll
  for (int g = 0; g < NS - 1; ++g) issue(g);
  for (int64_t kt = 0; kt < nk; ++kt) {
    wait_vmcnt<(NS - 2) * D>();  // this wave's loads of tile kt have landed
    __builtin_amdgcn_s_barrier();  // ... every wave's, and every wave is done with tile kt - 1
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    issue(kt + NS - 1);           // into the stage tile kt - 1 used
    compute(smem + static_cast<int>(kt % NS) * C::STAGE);
  }
  wait_vmcnt<0>();  // the re-reads past the last tile
  __syncthreads();
}

// Plain epilogue staged through LDS.  The accumulator layout gives each lane 4 consecutive outputs
// of one row, so direct stores cover 32 rows x 16 bytes per instruction; instead each wave writes
// one 32-row slab of its (already scaled and rounded) outputs into a private LDS buffer and reads
// it back as 16-byte row-contiguous chunks, so a store instruction covers whole row segments.
// Output values are the same as the direct path's.  Needs a 16-byte aligned output and row pitch.
// LDS bytes the staged epilogue of NWV waves needs with JU 32-column tiles per slab.
template <int NWV, int JU, int OUT_DT>
constexpr int epi32_bytes() {
  return NWV * 32 * (JU * 32 * (OUT_DT == kBF16 ? 2 : 4) + 16);
}

template <int NWV, int TM, int TN, int OUT_DT, int AVAIL, bool GATES>
__device__ __forceinline__ void epi32_plain_staged(const LinearArgs& a, const v16i (&acc)[TM][TN], const float (&sx)[TM],
                                                   const int32_t (&rsum)[TM], float cws, int64_t m0, int64_t n0,
                                                   int wm, int wn, char* smem) {
  constexpr int ES = OUT_DT == kBF16 ? 2 : 4;
  constexpr int JU = epi32_bytes<NWV, TN, OUT_DT>() <= AVAIL ? TN : 1;  // 32-col tiles per slab
  constexpr int RB = JU * 32 * ES;   // bytes of one staged row
  constexpr int PITCH = RB + 16;     // padded so the column-wise staging stores spread over the banks
  constexpr int CPR = RB / 16;       // 16-byte chunks per row
  constexpr int VPC = 16 / ES;       // outputs per chunk
  static_assert(NWV * 32 * PITCH <= AVAIL, "staging buffers exceed the LDS given");
  static_assert((32 * CPR) % 64 == 0, "chunks must divide over the wave");
  const int lane = threadIdx.x & 63;
  char* wb = smem + (threadIdx.x >> 6) * 32 * PITCH;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const float inv = 1.0f / sx[i];
    const int64_t mb = m0 + (wm * TM + i) * 32;
#pragma unroll
    for (int jb = 0; jb < TN; jb += JU) {
      lds_barrier();  // the buffer's previous contents (or the last K tile) are consumed
#pragma unroll
      for (int jj = 0; jj < JU; ++jj) {
        const int64_t nt = n0 + (wn * TN + jb + jj) * 32;  // the 32-column tile's first column
        const int kind = GATES ? gate_region(a, nt) : 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = (static_cast<float>(acc[i][jb + jj][4 * g + r] - rsum[i]) * inv) * cws;
          if constexpr (GATES) gate_act4<OUT_DT>(a, kind, nt + 8 * g + 4 * (lane >> 5), v);
          char* p = wb + (lane & 31) * PITCH + (jj * 32 + 8 * g + 4 * (lane >> 5)) * ES;
          if constexpr (OUT_DT == kBF16)
            *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
          else
            *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
      lds_barrier();
      const int64_t nb = n0 + (wn * TN + jb) * 32;
#pragma unroll
      for (int it = 0; it < 32 * CPR / 64; ++it) {
        const int idx = it * 64 + lane;
        const int row = idx / CPR, ch = idx % CPR;
        const int64_t m = mb + row, n = nb + ch * VPC;
        if (m >= a.M || n >= a.N) continue;
        const uint4 d = *reinterpret_cast<const uint4*>(wb + row * PITCH + ch * 16);
        char* dst = static_cast<char*>(a.out) + (m * a.ldo + n) * ES;
        if (n + VPC <= a.N) {
          *reinterpret_cast<uint4*>(dst) = d;
        } else {
          const uint32_t wd[4] = {d.x, d.y, d.z, d.w};
          for (int e = 0; e < a.N - n; ++e) {
            if constexpr (OUT_DT == kBF16)
              reinterpret_cast<uint16_t*>(dst)[e] = static_cast<uint16_t>(wd[e >> 1] >> (16 * (e & 1)));
            else
              reinterpret_cast<uint32_t*>(dst)[e] = wd[e];
          }
        }
      }
    }
  }
}

// NS == 0: register-staged main loop (two LDS stages); NS >= 2: direct-to-LDS loads into NS stages.
// One output tile at (m0, n0); smem holds SMEM bytes (at least the tile's stages).
template <int WM, int WN, int TM, int TN, int EPI, int OUT_DT, int NS, int SMEM>
__device__ __forceinline__ void mfma32_tile(const LinearArgs& a, int64_t m0, int64_t n0, char* smem) {
  using C = Cfg32<WM, WN, TM, TN>;
  static_assert((NS == 0 ? 2 : NS) * C::STAGE <= SMEM, "tile stages exceed the LDS given");
  v16i acc0[TM][TN], acc1[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      acc0[i][j] = v16i{};
      acc1[i][j] = v16i{};
    }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int wm = w / WN, wn = w % WN;
  const LinearOperand& o0 = a.op[0];
  const LinearOperand& o1 = a.op[1];
  const bool plain = (EPI == kEpiStore || EPI == kEpiGates) && !o0.c_w_per_row && !a.bias && !a.acc_dump;
  float sx[TM], sx1[TM];
  int32_t rsum[TM], rs1[TM];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + (wm * TM + i) * 32 + (lane & 31);
    const int64_t mc = m < a.M ? m : a.M - 1;
    sx[i] = o0.s_x[mc];
    rsum[i] = o0.rowsum[mc];
    if constexpr (epi_dual(EPI)) {
      sx1[i] = o1.s_x[mc];
      rs1[i] = o1.rowsum[mc];
    }
  }
  const float cws = o0.c_w[0];
  const float cws1 = epi_dual(EPI) ? o1.c_w[0] : 0.0f;
  if constexpr (NS == 0) {
    mfma32_mainloop<C, WN, TM, TN>(a.op[0], a.M, a.N, m0, n0, a.Kp, acc0, smem);
    if constexpr (epi_dual(EPI)) mfma32_mainloop<C, WN, TM, TN>(a.op[1], a.M, a.N, m0, n0, a.Kp, acc1, smem);
  } else {
    mfma32d_mainloop<C, WN, TM, TN, NS>(a.op[0], a.M, a.N, m0, n0, a.Kp, acc0, smem);
    if constexpr (epi_dual(EPI))
      mfma32d_mainloop<C, WN, TM, TN, NS>(a.op[1], a.M, a.N, m0, n0, a.Kp, acc1, smem);
  }

  const bool vout = vec4_ok<OUT_DT>(a.out, a.ldo);
  // the staged epilogue needs one 32-column slab per wave in the tile's LDS (else the direct stores)
  if constexpr (epi32_bytes<WM * WN, 1, OUT_DT>() <= SMEM) {
    if (plain && reinterpret_cast<uintptr_t>(a.out) % 16 == 0 && (a.ldo * (OUT_DT == kBF16 ? 2 : 4)) % 16 == 0) {
      epi32_plain_staged<WM * WN, TM, TN, OUT_DT, SMEM, EPI == kEpiGates>(a, acc0, sx, rsum, cws, m0, n0, wm, wn,
                                                                        smem);
      return;
    }
  }
  if (plain) {
    const int nrem = static_cast<int>(std::min<int64_t>(a.N - n0, C::BN));
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = m0 + (wm * TM + i) * 32 + (lane & 31);
      if (m >= a.M) continue;
      const float inv = 1.0f / sx[i];
      char* orow = static_cast<char*>(a.out) + (m * a.ldo + n0) * (OUT_DT == kBF16 ? 2 : 4);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int kind = EPI == kEpiGates ? gate_region(a, n0 + (wn * TN + j) * 32) : 0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int nb = (wn * TN + j) * 32 + 8 * g + 4 * (lane >> 5);
          if (nb >= nrem) continue;
          float v[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = (static_cast<float>(acc0[i][j][4 * g + r] - rsum[i]) * inv) * cws;
          if constexpr (EPI == kEpiGates) gate_act4<OUT_DT>(a, kind, n0 + nb, v);
          if (vout && nb + 4 <= nrem) {
            store4<OUT_DT>(orow, nb, v, true);
          } else {
            for (int r = 0; r < 4 && nb + r < nrem; ++r) st<OUT_DT>(orow, nb + r, v[r]);
          }
        }
      }
    }
    return;
  }
  // Generic epilogue.  The output-gate inputs of one 32 x 32 tile (four groups of four columns per
  // lane) are requested together in straight-line code (indices clamped into range, raw bits) before
  // any is used, so the tile waits for memory once instead of once per group; second-operand row
  // scales and sums and per-tensor weight scales were read before the K loop.
  const bool vin = EPI == kEpiOutputGate && vec4_ok<OUT_DT>(a.local, a.ld_local) &&
                   vec4_ok<OUT_DT>(a.gate, a.ld_gate) && a.N % 4 == 0;
  constexpr int es = OUT_DT == kBF16 ? 2 : 4;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = m0 + (wm * TM + i) * 32 + (lane & 31), mc = m < a.M ? m : a.M - 1;
    const float inv0 = 1.0f / sx[i];
    const float inv1 = epi_dual(EPI) ? 1.0f / sx1[i] : 0.0f;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      uint32_t lo[4][4], gt[4][4];
      if constexpr (EPI == kEpiOutputGate) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int64_t nb = n0 + (wn * TN + j) * 32 + 8 * g + 4 * (lane >> 5);
          if (vin) {  // whole groups of four: a group past N re-reads the last one
            const int64_t nv = nb < a.N ? nb : a.N - 4;
            const char* pl = static_cast<const char*>(a.local) + (mc * a.ld_local + nv) * es;
            const char* pg = static_cast<const char*>(a.gate) + (mc * a.ld_gate + nv) * es;
#pragma unroll
            for (int q = 0; q < es / 2; ++q) {  // bf16: one 8-byte load, f32: two
              const uint2 wl = reinterpret_cast<const uint2*>(pl)[q], wg = reinterpret_cast<const uint2*>(pg)[q];
              lo[g][2 * q] = wl.x;
              lo[g][2 * q + 1] = wl.y;
              gt[g][2 * q] = wg.x;
              gt[g][2 * q + 1] = wg.y;
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int64_t n = nb + r < a.N ? nb + r : a.N - 1;
              lo[g][r] = ld_bits<OUT_DT>(a.local, mc * a.ld_local + n);
              gt[g][r] = ld_bits<OUT_DT>(a.gate, mc * a.ld_gate + n);
            }
          }
        }
      }
      if (m >= a.M) continue;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t nb = n0 + (wn * TN + j) * 32 + 8 * g + 4 * (lane >> 5);
        if (nb >= a.N) continue;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t n = nb + r;
          const float cw0 = o0.c_w_per_row ? o0.c_w[n < a.N ? n : a.N - 1] : cws;
          const int32_t a0 = acc0[i][j][4 * g + r] - rsum[i];
          if (a.acc_dump && n < a.N) a.acc_dump[m * a.N + n] = a0;
          const float v0 = (static_cast<float>(a0) * inv0) * cw0;
          if constexpr (!epi_dual(EPI)) {  // (kEpiGates is always plain)
            v[r] = a.bias ? v0 + ld<OUT_DT>(a.bias, n < a.N ? n : a.N - 1) : v0;
          } else {
            const float cw1 = o1.c_w_per_row ? o1.c_w[n < a.N ? n : a.N - 1] : cws1;
            const float v1 = rnd<OUT_DT>((static_cast<float>(acc1[i][j][4 * g + r] - rs1[i]) * inv1) * cw1);
            float lv = 0.0f, gv = 0.0f;
            if constexpr (EPI == kEpiOutputGate) {
              if (vin && OUT_DT == kBF16) {
                const uint32_t wl = lo[g][r >> 1], wg = gt[g][r >> 1];
                lv = __uint_as_float(r & 1 ? wl & 0xffff0000u : wl << 16);
                gv = __uint_as_float(r & 1 ? wg & 0xffff0000u : wg << 16);
              } else {
                lv = from_bits<OUT_DT>(lo[g][r]);
                gv = from_bits<OUT_DT>(gt[g][r]);
              }
            }
            v[r] = dual_epi<EPI, OUT_DT>(rnd<OUT_DT>(v0), v1, lv, gv);
          }
        }
        if (nb + 3 < a.N) {
          store4<OUT_DT>(a.out, m * a.ldo + nb, v, vout);
        } else {
          for (int r = 0; r < 4 && nb + r < a.N; ++r) st<OUT_DT>(a.out, m * a.ldo + nb + r, v[r]);
        }
      }
    }
  }
}

template <int WM, int WN, int TM, int TN, int EPI, int OUT_DT, int NS = 0>
__global__ __launch_bounds__(WM* WN * 64) void mfma32_kernel(LinearArgs a) {
  using C = Cfg32<WM, WN, TM, TN>;
  constexpr int SMEM = (NS == 0 ? 2 : NS) * C::STAGE;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  int64_t tm, tn;
  xcd_tile((a.M + C::BM - 1) / C::BM, (a.N + C::BN - 1) / C::BN, tm, tn);
  mfma32_tile<WM, WN, TM, TN, EPI, OUT_DT, NS, SMEM>(a, tm * C::BM, tn * C::BN, smem);
}

// Plain product whose 128x256 tiles would run in more rounds than the CUs hold (the SISO in_proj, 640
// tiles): columns [0, nA) in 128x256 tiles, two per CU, and the remaining N - nA columns in 128x128
// tiles launched after them, so the last round runs half-size tiles on more CUs.  Both use two
// direct-to-LDS stages and eight waves; TMB = 32-row MFMA tiles per wave of a tail tile (2: 128 rows).
template <int OUT_DT, int TMB, int EPI>
__global__ __launch_bounds__(512) void mfma32_split_kernel(LinearArgs a, int64_t nA) {
  using CA = Cfg32<2, 4, 2, 2>;
  using CB = Cfg32<2, 4, TMB, 1>;
  constexpr int SMEM = 2 * (CA::STAGE > CB::STAGE ? CA::STAGE : CB::STAGE);
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  const int64_t ntm = (a.M + CA::BM - 1) / CA::BM, ntnA = nA / CA::BN, tilesA = ntm * ntnA;
  int64_t tm, tn;
  if (static_cast<int64_t>(blockIdx.x) < tilesA) {
    xcd_tile_of(blockIdx.x, ntm, ntnA, tm, tn);
    mfma32_tile<2, 4, 2, 2, EPI, OUT_DT, 2, SMEM>(a, tm * CA::BM, tn * CA::BN, smem);
  } else {
    xcd_tile_of(blockIdx.x - tilesA, (a.M + CB::BM - 1) / CB::BM, (a.N - nA + CB::BN - 1) / CB::BN, tm, tn);
    mfma32_tile<2, 4, TMB, 1, EPI, OUT_DT, 2, SMEM>(a, tm * CB::BM, nA + tn * CB::BN, smem);
  }
}

// ---------------------------------------------------------------------------
// Output gate over whole rows: a workgroup owns 16 rows and all N = d_model columns (NW waves side
// by side, NCT 16-column tiles each), so after y = local + sigmoid(gate)*state_proj + ent_proj it
// can quantize y per token for out_proj without writing y.  Every global operand of the epilogue
// (local, gate, s_x, rowsum) is requested before the K loop and kept as raw bits, so the whole
// workgroup's memory traffic is in flight at once; the K loop runs two k-steps per iteration on
// ping-pong registers so each MFMA group waits only for its own operands.
// ---------------------------------------------------------------------------

// Raw 32-bit words holding four consecutive epilogue values of one row: two bf16 pairs when the
// row can be read with one 8-byte load, else one word per value.
template <int DT, bool VEC>
struct EpRaw {
  static constexpr int W = (DT == kBF16 && VEC) ? 2 : 4;
};

// Columns past N read the last valid ones (their results are never stored).
template <int DT, bool VEC>
__device__ __forceinline__ void ep_load(const void* base, int64_t ld, int64_t m, int64_t nb, int64_t N,
                                        uint32_t (&raw)[EpRaw<DT, VEC>::W]) {
  if constexpr (VEC) {
    const int64_t c = nb < N ? nb : N - 4;  // N % 4 == 0
    if constexpr (DT == kBF16) {
      const v2u x = *reinterpret_cast<const v2u*>(static_cast<const uint16_t*>(base) + m * ld + c);
      raw[0] = x.x;
      raw[1] = x.y;
    } else {
      const v4i x = *reinterpret_cast<const v4i*>(static_cast<const float*>(base) + m * ld + c);
#pragma unroll
      for (int r = 0; r < 4; ++r) raw[r] = static_cast<uint32_t>(x[r]);
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t c = nb + r < N ? nb + r : N - 1;
      if constexpr (DT == kBF16)
        raw[r] = static_cast<const uint16_t*>(base)[m * ld + c];
      else
        raw[r] = static_cast<const uint32_t*>(base)[m * ld + c];
    }
  }
}

template <int DT, bool VEC>
__device__ __forceinline__ float ep_get(const uint32_t (&raw)[EpRaw<DT, VEC>::W], int r) {
  if constexpr (DT == kF32) {
    return __uint_as_float(raw[r]);
  } else if constexpr (VEC) {
    return __uint_as_float((r & 1) ? (raw[r >> 1] & 0xffff0000u) : (raw[r >> 1] << 16));
  } else {
    return __uint_as_float(raw[r] << 16);
  }
}

// One k-step of both operands for the lanes' row (A: 16 code bytes) and tiles (B: a packed dword).
template <int NCT>
__device__ __forceinline__ void rowq_load(const LinearArgs& a, int64_t mc, int64_t col0, int lane, int64_t ks,
                                          v4i& x0, v4i& x1, uint32_t (&w0)[NCT], uint32_t (&w1)[NCT]) {
  const LinearOperand& o0 = a.op[0];
  const LinearOperand& o1 = a.op[1];
  const int64_t ko = 64 * ks + 16 * (lane >> 4);
  x0 = *reinterpret_cast<const v4i*>(o0.q + mc * o0.ldq + ko);
  x1 = *reinterpret_cast<const v4i*>(o1.q + mc * o1.ldq + ko);
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    const int64_t n = col0 + 16 * j + (lane & 15);
    const int64_t nc = n < a.N ? n : a.N - 1;
    w0[j] = *reinterpret_cast<const uint32_t*>(o0.w + nc * o0.ldw + ko / 4);
    w1[j] = *reinterpret_cast<const uint32_t*>(o1.w + nc * o1.ldw + ko / 4);
  }
}

template <int NCT>
__device__ __forceinline__ void rowq_mma(v4i (&acc0)[NCT], v4i (&acc1)[NCT], const v4i& x0, const v4i& x1,
                                         const uint32_t (&w0)[NCT], const uint32_t (&w1)[NCT]) {
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    acc0[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack_frag(w0[j]), x0, acc0[j], 0, 0, 0);
    acc1[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack_frag(w1[j]), x1, acc1[j], 0, 0, 0);
  }
}

// y = local + sigmoid(gate) * state_proj + ent_proj in the reference's op order (tesm.py:1256-1260),
// every op rounded to the layer dtype; entries outside the matrix are 0.  PER_ROW: c_w0 / c_w1
// index per output column, else they point at one scalar each.
template <int NCT, int DT, bool VEC, bool PER_ROW>
__device__ __forceinline__ void rowq_gate(const LinearArgs& a, const uint32_t (&lraw)[NCT][EpRaw<DT, VEC>::W],
                                          const uint32_t (&graw)[NCT][EpRaw<DT, VEC>::W], const v4i (&acc0)[NCT],
                                          const v4i (&acc1)[NCT], int32_t rs0, int32_t rs1, float inv0, float inv1,
                                          const float* c_w0, const float* c_w1, bool mok, int64_t col0, int lane,
                                          float (&y)[NCT][4]) {
  const float cws0 = c_w0[0], cws1 = c_w1[0];
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t n = col0 + 16 * j + 4 * (lane >> 4) + r;
      const int64_t nc = n < a.N ? n : a.N - 1;
      const float cw0 = PER_ROW ? c_w0[nc] : cws0;
      const float cw1 = PER_ROW ? c_w1[nc] : cws1;
      const float sp = rnd<DT>((static_cast<float>(acc0[j][r] - rs0) * inv0) * cw0);
      const float ep = rnd<DT>((static_cast<float>(acc1[j][r] - rs1) * inv1) * cw1);
      const float g = rnd<DT>(sigmoidf_(ep_get<DT, VEC>(graw[j], r)));
      const float v = rnd<DT>(rnd<DT>(ep_get<DT, VEC>(lraw[j], r) + rnd<DT>(g * sp)) + ep);
      y[j][r] = (mok && n < a.N) ? v : 0.0f;
    }
  }
}

template <int NW, int NCT, int DT, bool VEC, int NKS>
__global__ __launch_bounds__(NW * 64) void gate_rowq_kernel(LinearArgs a, RowQuant o) {
  constexpr int RW = EpRaw<DT, VEC>::W;
  extern __shared__ __attribute__((aligned(16))) char lds_rowq[];
  int8_t* codes = reinterpret_cast<int8_t*>(lds_rowq);                          // [16][ldq]
  float* red = reinterpret_cast<float*>(lds_rowq + 16 * o.ldq);                 // [16 rows][NW waves]
  int32_t* redi = reinterpret_cast<int32_t*>(red + 16 * NW);                   // [16 rows][NW waves]
  float* cwl = reinterpret_cast<float*>(redi + 16 * NW);                       // [2][N] per-row scales
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 16;
  const int64_t col0 = static_cast<int64_t>(w) * NCT * 16;
  const LinearOperand& o0 = a.op[0];
  const LinearOperand& o1 = a.op[1];
  const int row = lane & 15;  // the activation row this lane feeds and the output row it holds
  const int64_t m = m0 + row;
  const bool mok = m < a.M;
  const int64_t mc = mok ? m : a.M - 1;
  const int64_t nks = a.Kp / 64;  // even: Kp is a multiple of 128
  const bool per_row = o0.c_w_per_row || o1.c_w_per_row;

  if (per_row) {
    for (int64_t i = tid; i < a.N; i += NW * 64) {
      cwl[i] = o0.c_w_per_row ? o0.c_w[i] : o0.c_w[0];
      cwl[a.N + i] = o1.c_w_per_row ? o1.c_w[i] : o1.c_w[0];
    }
  }
  // epilogue operands first, as raw bits: nothing waits on them before the K loop is done
  uint32_t lraw[NCT][RW], graw[NCT][RW];
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    const int64_t nb = col0 + 16 * j + 4 * (lane >> 4);
    ep_load<DT, VEC>(a.local, a.ld_local, mc, nb, a.N, lraw[j]);
    ep_load<DT, VEC>(a.gate, a.ld_gate, mc, nb, a.N, graw[j]);
  }
  const float sx0 = o0.s_x[mc], sx1 = o1.s_x[mc];
  const int32_t rs0 = o0.rowsum[mc], rs1 = o1.rowsum[mc];
  const float cws0 = o0.c_w[0], cws1 = o1.c_w[0];
  for (int64_t i = tid; i < 16 * o.ldq / 16; i += NW * 64) reinterpret_cast<uint4*>(codes)[i] = make_uint4(0, 0, 0, 0);

  v4i acc0[NCT], acc1[NCT];
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    acc0[j] = v4i{0, 0, 0, 0};
    acc1[j] = v4i{0, 0, 0, 0};
  }
  if constexpr (NKS > 0) {
    // the whole K extent at once (NKS == Kp / 64): one round trip for all of the wave's operands
    v4i x0[NKS], x1[NKS];
    uint32_t w0[NKS][NCT], w1[NKS][NCT];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) rowq_load<NCT>(a, mc, col0, lane, ks, x0[ks], x1[ks], w0[ks], w1[ks]);
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the first MFMA
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) rowq_mma<NCT>(acc0, acc1, x0[ks], x1[ks], w0[ks], w1[ks]);
  } else {
    v4i xa0, xa1, xb0, xb1;
    uint32_t wa0[NCT], wa1[NCT], wb0[NCT], wb1[NCT];
    rowq_load<NCT>(a, mc, col0, lane, 0, xa0, xa1, wa0, wa1);
    for (int64_t ks = 0; ks < nks; ks += 2) {
      rowq_load<NCT>(a, mc, col0, lane, ks + 1, xb0, xb1, wb0, wb1);
      rowq_mma<NCT>(acc0, acc1, xa0, xa1, wa0, wa1);
      // the last iteration re-reads k-step ks + 1 instead of branching (the values are unused)
      rowq_load<NCT>(a, mc, col0, lane, ks + 2 < nks ? ks + 2 : ks + 1, xa0, xa1, wa0, wa1);
      rowq_mma<NCT>(acc0, acc1, xb0, xb1, wb0, wb1);
    }
  }
  if (per_row) __syncthreads();

  // epilogue: lane holds row m, columns col0 + 16j + 4*(lane/16) + r
  const float inv0 = 1.0f / sx0, inv1 = 1.0f / sx1;
  float y[NCT][4];
  if (per_row)
    rowq_gate<NCT, DT, VEC, true>(a, lraw, graw, acc0, acc1, rs0, rs1, inv0, inv1, cwl, cwl + a.N, mok, col0, lane, y);
  else
    rowq_gate<NCT, DT, VEC, false>(a, lraw, graw, acc0, acc1, rs0, rs1, inv0, inv1, &cws0, &cws1, mok, col0, lane, y);
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
#pragma unroll
    for (int r = 0; r < 4; ++r) mx = fmaxf(mx, fabsf(y[j][r]));
  }
  if (o.y && mok) {
    const bool vout = vec4_ok<DT>(o.y, o.ldy);
#pragma unroll
    for (int j = 0; j < NCT; ++j) {
      const int64_t nb = col0 + 16 * j + 4 * (lane >> 4);
      if (vout && nb + 3 < a.N) {
        store4<DT>(o.y, m * o.ldy + nb, y[j], true);
      } else {
        for (int r = 0; r < 4 && nb + r < a.N; ++r) st<DT>(o.y, m * o.ldy + nb + r, y[j][r]);
      }
    }
  }
  // row max over the 4 lanes sharing the row, then over the NW waves
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (lane < 16) red[row * NW + w] = mx;
  __syncthreads();
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) amax = fmaxf(amax, red[row * NW + i]);
  const float sc = act_scale<DT>(amax, o.eps);
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
  if (lane < 16) redi[row * NW + w] = sum;
  __syncthreads();
  if (tid < 16 && m0 + tid < a.M) {
    float am = 0.0f;
    int32_t rsum = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      am = fmaxf(am, red[tid * NW + i]);
      rsum += redi[tid * NW + i];
    }
    o.s[m0 + tid] = act_scale<DT>(am, o.eps);
    o.rs[m0 + tid] = rsum;
  }
  const int64_t chunks = o.ldq / 16;
  for (int r = w; r < 16; r += NW) {
    if (m0 + r >= a.M) continue;
    for (int64_t ck = lane; ck < chunks; ck += 64)
      reinterpret_cast<uint4*>(o.q + (m0 + r) * o.ldq)[ck] = reinterpret_cast<const uint4*>(codes + r * o.ldq)[ck];
  }
}

// ---------------------------------------------------------------------------
// Persistent output gate with both packed weight matrices resident in LDS (gfx950: 160 KB per
// workgroup).  Each workgroup stages state_proj and ent_proj once with coalesced 16-byte loads and
// then walks 16-row tiles blockIdx.x, blockIdx.x + gridDim.x, ...; the next tile's activation codes
// (one 16-byte piece per thread, staged through LDS) and local/gate operands are requested before
// the current tile is computed.
//
// Staged weight row n of operand p sits at (p * N + n) * RS bytes, RS = 16 * NKS + 16; dword
// q * NKS + ks of a row holds codes 64 ks + 16 q .. + 15, so one lane reads all its k-steps with
// wide LDS loads and a 16-lane row group covers all 64 banks once.  Activation rows are staged at
// a pitch of Kp + 16 bytes for the same reason.
// ---------------------------------------------------------------------------
template <int NKS>
struct RowqLds {
  static constexpr int RS = 16 * NKS + 16;           // staged weight row pitch
  static constexpr int ARS = 64 * NKS + 16;          // staged activation row pitch
  static constexpr int ABUF = 2 * 16 * ARS;          // one tile of both operands
};

inline int64_t rowq_lds_bytes(int64_t N, int64_t nks, int64_t ldq, int nw) {
  const int64_t stage = nks <= 4 ? 0 : 2 * N * (16 * nks + 16);  // register-resident weights for K <= 256
  return stage + 2 * 2 * 16 * (64 * nks + 16) + 16 * (ldq + 16) + 2 * 2 * 16 * nw * 4 + 2 * N * 4;
}

template <int NCT, int AC, int RW>
struct RowqIn {
  v4i ac[AC];                          // this thread's share of the tile's activation codes
  uint32_t lr[NCT][RW], gr[NCT][RW];   // raw local / gate values of the lane's row
  float sx0, sx1;
  int32_t rs0, rs1;
};

// Requests for tile t; rows past M read the last row (never stored).
template <int NW, int NCT, int NKS, int DT, int AC>
__device__ __forceinline__ void rowq_in_load(const LinearArgs& a, int64_t t, int64_t col0, int tid,
                                             RowqIn<NCT, AC, EpRaw<DT, true>::W>& in) {
  const int lane = tid & 63;
  const int64_t m0 = t * 16;
  const int64_t m = m0 + (lane & 15);
  const int64_t mc = m < a.M ? m : a.M - 1;
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    int g = tid + i * NW * 64;
    g = g < 128 * NKS ? g : 128 * NKS - 1;
    const int p = g / (64 * NKS), rem = g - p * 64 * NKS;
    const int r = rem / (4 * NKS), c = rem - r * 4 * NKS;
    const int64_t mr = m0 + r < a.M ? m0 + r : a.M - 1;
    const LinearOperand& op = a.op[0];
    const int8_t* src = p == 0 ? op.q + mr * op.ldq : a.op[1].q + mr * a.op[1].ldq;
    in.ac[i] = *reinterpret_cast<const v4i*>(src + 16 * c);
  }
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    const int64_t nb = col0 + 16 * j + 4 * (lane >> 4);
    ep_load<DT, true>(a.local, a.ld_local, mc, nb, a.N, in.lr[j]);
    ep_load<DT, true>(a.gate, a.ld_gate, mc, nb, a.N, in.gr[j]);
  }
  in.sx0 = a.op[0].s_x[mc];
  in.sx1 = a.op[1].s_x[mc];
  in.rs0 = a.op[0].rowsum[mc];
  in.rs1 = a.op[1].rowsum[mc];
}

// NKS consecutive dwords of staged LDS (16-byte aligned when NKS % 4 == 0, else 8-byte aligned).
template <int NKS>
__device__ __forceinline__ void lds_frag(const char* p, uint32_t (&f)[NKS]) {
  if constexpr (NKS % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NKS / 4; ++i) {
      const v4i v = reinterpret_cast<const v4i*>(p)[i];
#pragma unroll
      for (int r = 0; r < 4; ++r) f[4 * i + r] = static_cast<uint32_t>(v[r]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NKS / 2; ++i) {
      const v2u v = reinterpret_cast<const v2u*>(p)[i];
      f[2 * i] = v.x;
      f[2 * i + 1] = v.y;
    }
  }
}

struct RowqShared {
  const char* wl;     // staged weights
  char* abuf;         // staged activation tile (this tile's buffer)
  int8_t* codes;      // [16][ldq]
  float* red;         // [16][NW] (this tile's buffer)
  int32_t* redi;      // [16][NW] (this tile's buffer)
  const float* cwl;   // [2][N] output scale of every column (c_w, or its one scalar repeated)
};

// Packed-weight fragments of the lane's columns for the register-resident variant (NKS <= 4).  The
// lanes of group q take the 16-code groups q NKS .. q NKS + NKS - 1 of their column (k-step ks: group
// q NKS + ks, for weights and activation codes alike), so each lane's fragments are one contiguous
// load and a column's four lanes read its packed row whole.
template <int NCT, int NKS>
struct RowqW {
  uint32_t w0[NCT][NKS], w1[NCT][NKS];
};

template <int NW, int NCT, int DT, int NKS, int AC, bool RW = false>
__device__ __forceinline__ void rowq_tile(const LinearArgs& a, const RowQuant& o, int64_t t,
                                          const RowqIn<NCT, AC, EpRaw<DT, true>::W>& in, const RowqShared& sh,
                                          int tid, const RowqW<NCT, NKS>* rw = nullptr) {
  using L = RowqLds<NKS>;
  // all in-tile indices fit 32 bits: N <= 1024 and the LDS is 160 KB
  const int N = static_cast<int>(a.N);
  const int cp = static_cast<int>(o.ldq) + 16;  // staged code row pitch (16 rows spread over all banks)
  const int lane = tid & 63, w = tid >> 6, q = lane >> 4;
  const int col0 = w * NCT * 16;
  const int row = lane & 15;
  const int64_t m0 = t * 16;

  // activation tile into LDS, then each lane's row fragments for every k-step
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int g = tid + i * NW * 64;
    if (g >= 128 * NKS) continue;
    const int p = g / (64 * NKS), rem = g - p * 64 * NKS;
    const int r = rem / (4 * NKS), c = rem - r * 4 * NKS;
    *reinterpret_cast<v4i*>(sh.abuf + (p * 16 + r) * L::ARS + 16 * c) = in.ac[i];
  }
  __syncthreads();
  v4i x0[NKS], x1[NKS];
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const int kb = RW ? 16 * (q * NKS + ks) : 64 * ks + 16 * q;  // the k-step's code group of lane group q
    x0[ks] = *reinterpret_cast<const v4i*>(sh.abuf + row * L::ARS + kb);
    x1[ks] = *reinterpret_cast<const v4i*>(sh.abuf + (16 + row) * L::ARS + kb);
  }

  // per 16-column tile: both products, then y = local + sigmoid(gate) * state_proj + ent_proj in the
  // reference's op order (tesm.py:1256-1260), every op rounded to the layer dtype.  Rows past M
  // compute finite values from clamped operands and are never stored.
  const float inv0 = 1.0f / in.sx0, inv1 = 1.0f / in.sx1;
  float y[NCT][4];
  float mx = 0.0f;
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    const int n = col0 + 16 * j + row;
    const int nc = n < N ? n : N - 1;
    uint32_t f0[NKS], f1[NKS];
    if constexpr (RW) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        f0[ks] = rw->w0[j][ks];
        f1[ks] = rw->w1[j][ks];
        // opaque copies: the unpacking below stays per tile instead of being hoisted out of the tile
        // loop as 4x as many live registers
        asm volatile("" : "+v"(f0[ks]));
        asm volatile("" : "+v"(f1[ks]));
      }
    } else {
      lds_frag<NKS>(sh.wl + nc * L::RS + q * NKS * 4, f0);
      lds_frag<NKS>(sh.wl + (N + nc) * L::RS + q * NKS * 4, f1);
    }
    v4i acc0 = v4i{0, 0, 0, 0}, acc1 = v4i{0, 0, 0, 0};
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      acc0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack_frag(f0[ks]), x0[ks], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(unpack_frag(f1[ks]), x1[ks], acc1, 0, 0, 0);
    }
    const int nb = col0 + 16 * j + 4 * q;
    const int nbc = nb < N ? nb : N - 4;  // N % 4 == 0
    const float4 cw0 = *reinterpret_cast<const float4*>(sh.cwl + nbc);
    const float4 cw1 = *reinterpret_cast<const float4*>(sh.cwl + N + nbc);
    const float c0[4] = {cw0.x, cw0.y, cw0.z, cw0.w}, c1[4] = {cw1.x, cw1.y, cw1.z, cw1.w};
    const bool nok = nb < N;  // N % 4 == 0: the lane's 4 columns are all in range or all out
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float sp = rnd<DT>((static_cast<float>(acc0[r] - in.rs0) * inv0) * c0[r]);
      const float ep = rnd<DT>((static_cast<float>(acc1[r] - in.rs1) * inv1) * c1[r]);
      const float g = rnd<DT>(sigmoidf_(ep_get<DT, true>(in.gr[j], r)));
      const float v = rnd<DT>(rnd<DT>(ep_get<DT, true>(in.lr[j], r) + rnd<DT>(g * sp)) + ep);
      y[j][r] = nok ? v : 0.0f;
      mx = fmaxf(mx, fabsf(y[j][r]));
    }
  }
  const int64_t m = m0 + row;
  if (o.y && m < a.M) {
    const bool vout = vec4_ok<DT>(o.y, o.ldy);
#pragma unroll
    for (int j = 0; j < NCT; ++j) {
      const int nb = col0 + 16 * j + 4 * q;
      if (vout && nb < N) {
        store4<DT>(o.y, m * o.ldy + nb, y[j], true);
      } else {
        for (int r = 0; r < 4 && nb + r < N; ++r) st<DT>(o.y, m * o.ldy + nb + r, y[j][r]);
      }
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (lane < 16) sh.red[row * NW + w] = mx;
  __syncthreads();
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) amax = fmaxf(amax, sh.red[row * NW + i]);
  const float sc = act_scale<DT>(amax, o.eps);
  // layout 1: column n = 16 g + 4 q + r sits at byte 16 g + 4 r + q of its row
  int sum = 0;
  int8_t* crow = sh.codes + row * cp + col0 + q;
#pragma unroll
  for (int j = 0; j < NCT; ++j) {
    if (col0 + 16 * j + 4 * q >= N) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int qv = act_code<DT>(y[j][r], sc);
      crow[16 * j + 4 * r] = static_cast<int8_t>(qv);
      sum += qv;
    }
  }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  if (lane < 16) sh.redi[row * NW + w] = sum;
  __syncthreads();
  if (tid < 16 && m0 + tid < a.M) {
    float am = 0.0f;
    int32_t rsum = 0;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      am = fmaxf(am, sh.red[tid * NW + i]);
      rsum += sh.redi[tid * NW + i];
    }
    o.s[m0 + tid] = act_scale<DT>(am, o.eps);
    o.rs[m0 + tid] = rsum;
  }
  const int chunks = static_cast<int>(o.ldq / 16);
  for (int r = w; r < 16; r += NW) {
    if (m0 + r >= a.M) continue;
    uint4* dst = reinterpret_cast<uint4*>(o.q + (m0 + r) * o.ldq);
    const uint4* src = reinterpret_cast<const uint4*>(sh.codes + r * cp);
    for (int ck = lane; ck < chunks; ck += 64) dst[ck] = src[ck];
  }
}

// NKS <= 4 (K <= 256): each wave's packed-weight fragments (its NCT column tiles of both products, 2 NCT
// NKS dwords per lane) stay in registers for the whole kernel, read straight from global memory;
// otherwise both weight matrices are staged once per workgroup in LDS.
template <int NKS>
constexpr bool rowq_reg_weights() {
  return NKS <= 4;
}

template <int NW, int NCT, int DT, int NKS>
__global__ __launch_bounds__(NW * 64) void gate_rowq_lds_kernel(LinearArgs a, RowQuant o, int64_t ntiles) {
  using L = RowqLds<NKS>;
  constexpr bool RW = rowq_reg_weights<NKS>();
  constexpr int NT = NW * 64;
  constexpr int SB = RW ? 1 : (2 * NW * NCT * 16 * NKS + NT - 1) / NT;  // staged weight chunks per thread
  constexpr int AC = (128 * NKS + NT - 1) / NT;                          // activation chunks per thread per tile
  using In = RowqIn<NCT, AC, EpRaw<DT, true>::W>;
  extern __shared__ __attribute__((aligned(16))) char lds_rowq[];
  char* wl = lds_rowq;                                                    // [2][N][RS] (LDS weights only)
  char* abuf = wl + (RW ? 0 : 2 * a.N * L::RS);                           // [2 tiles][2][16][ARS]
  int8_t* codes = reinterpret_cast<int8_t*>(abuf + 2 * L::ABUF);          // [16][ldq + 16]
  float* red = reinterpret_cast<float*>(codes + 16 * (o.ldq + 16));       // [2 tiles][16][NW]
  int32_t* redi = reinterpret_cast<int32_t*>(red + 2 * 16 * NW);         // [2 tiles][16][NW]
  float* cwl = reinterpret_cast<float*>(redi + 2 * 16 * NW);             // [2][N]
  const int tid = threadIdx.x;
  const int64_t col0 = static_cast<int64_t>(tid >> 6) * NCT * 16;

  // weights: every load first (registers, or the LDS stage), then this workgroup's first tile, then
  // the LDS writes
  RowqW<NCT, NKS> rw;
  v4i sb[SB];
  const int64_t total = 2 * a.N * NKS;
  if constexpr (RW) {
    // lane (q, row) of column tile j: column col0 + 16 j + row, dwords q NKS .. q NKS + NKS - 1 of its row
    const int lane = tid & 63, q = lane >> 4, row = lane & 15;
#pragma unroll
    for (int j = 0; j < NCT; ++j) {
      const int64_t n = col0 + 16 * j + row, nc = n < a.N ? n : a.N - 1;
      const uint32_t* p0 = reinterpret_cast<const uint32_t*>(a.op[0].w + nc * a.op[0].ldw) + q * NKS;
      const uint32_t* p1 = reinterpret_cast<const uint32_t*>(a.op[1].w + nc * a.op[1].ldw) + q * NKS;
      if constexpr (NKS == 4) {
        const uint4 v0 = *reinterpret_cast<const uint4*>(p0), v1 = *reinterpret_cast<const uint4*>(p1);
        rw.w0[j][0] = v0.x, rw.w0[j][1] = v0.y, rw.w0[j][2] = v0.z, rw.w0[j][3] = v0.w;
        rw.w1[j][0] = v1.x, rw.w1[j][1] = v1.y, rw.w1[j][2] = v1.z, rw.w1[j][3] = v1.w;
      } else {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          rw.w0[j][ks] = p0[ks];
          rw.w1[j][ks] = p1[ks];
        }
      }
    }
  } else {
#pragma unroll
    for (int b = 0; b < SB; ++b) {
      const int64_t g = tid + static_cast<int64_t>(b) * NT;
      const int64_t gc = g < total ? g : total - 1;
      const int64_t pn = gc / NKS, c = gc - pn * NKS;  // pn = p * N + n
      const uint8_t* wp = pn < a.N ? a.op[0].w + pn * a.op[0].ldw : a.op[1].w + (pn - a.N) * a.op[1].ldw;
      sb[b] = *reinterpret_cast<const v4i*>(wp + 16 * c);
    }
  }
  RowqShared sh0, sh1;
  sh0.wl = sh1.wl = wl;
  sh0.abuf = abuf;
  sh1.abuf = abuf + L::ABUF;
  sh0.codes = sh1.codes = codes;
  sh0.red = red;
  sh1.red = red + 16 * NW;
  sh0.redi = redi;
  sh1.redi = redi + 16 * NW;
  sh0.cwl = sh1.cwl = cwl;
  In ta, tb;
  int64_t t = blockIdx.x;
  rowq_in_load<NW, NCT, NKS, DT, AC>(a, t, col0, tid, ta);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (!RW) {
#pragma unroll
    for (int b = 0; b < SB; ++b) {
      const int64_t g = tid + static_cast<int64_t>(b) * NT;
      if (g >= total) continue;
      const int64_t pn = g / NKS, c = g - pn * NKS;
      uint32_t* dst = reinterpret_cast<uint32_t*>(wl + pn * L::RS) + c;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) dst[qq * NKS] = static_cast<uint32_t>(sb[b][qq]);
    }
  }
  for (int64_t i = tid; i < a.N; i += NT) {
    cwl[i] = a.op[0].c_w_per_row ? a.op[0].c_w[i] : a.op[0].c_w[0];
    cwl[a.N + i] = a.op[1].c_w_per_row ? a.op[1].c_w[i] : a.op[1].c_w[0];
  }
  for (int64_t i = tid; i < (o.ldq + 16); i += NT) reinterpret_cast<uint4*>(codes)[i] = make_uint4(0, 0, 0, 0);
  // (the first tile's barrier after its activation staging also orders these LDS writes)

  // two tiles per iteration on ping-pong registers and LDS buffers; a prefetch past the end
  // re-reads the current tile
  for (;;) {
    const int64_t t1 = t + gridDim.x;
    rowq_in_load<NW, NCT, NKS, DT, AC>(a, t1 < ntiles ? t1 : t, col0, tid, tb);
    rowq_tile<NW, NCT, DT, NKS, AC, RW>(a, o, t, ta, sh0, tid, &rw);
    if (t1 >= ntiles) break;
    const int64_t t2 = t1 + gridDim.x;
    rowq_in_load<NW, NCT, NKS, DT, AC>(a, t2 < ntiles ? t2 : t1, col0, tid, ta);
    rowq_tile<NW, NCT, DT, NKS, AC, RW>(a, o, t1, tb, sh1, tid, &rw);
    if (t2 >= ntiles) break;
    t = t2;
  }
}

// ---------------------------------------------------------------------------
// Output gate on 32-row tiles (v_mfma_i32_32x32x32_i8).  A workgroup of NW waves owns 32 tokens and
// all N = d_model columns (wave w: NCT 32-column tiles from 32 NCT w), so it can quantize y per
// token for out_proj without writing y.  Per 32x32 product each unpacked weight dword serves 32
// tokens (twice the 16-row kernel's reuse), and the epilogue is cut to the operations the reference
// rounds (one conversion per bf16 rounding), codes written to LDS byte by byte in layout 1 (no VALU)
// and their sums formed with v_dot4 while the tile is copied out.
//
// Operands: weights are the MFMA's A operand (D rows = output columns), activation codes the B
// operand (D columns = tokens), so lane (t, h) holds token t and output columns 8 g + 4 h + r of each
// 32-column tile.  Lane half h takes the 16-code groups h NKS .. h NKS + NKS - 1 of a row (K step ks:
// group h NKS + ks, for both operands), so a lane's packed weight fragments are one contiguous read.
// ---------------------------------------------------------------------------
template <int NKS>
struct G32 {
  static constexpr int ARS = 32 * NKS + 16;  // staged activation row pitch: 16 rows span all banks
};

// bf16 local / gate are staged per wave in LDS (G32S: slab row pitch of NCT 32-column tiles)
template <int NCT>
struct G32S {
  // 16 NCT + 2 words: an odd multiple of two words, so the 32 rows of an 8-byte read hit 64 distinct banks
  static constexpr int SP = NCT * 64 + 8;
};

inline int64_t gate32_lds_bytes(int64_t Kp, int64_t ldq, int64_t nct, int nw, bool staged) {
  const int64_t slab = staged ? nw * 2 * 32 * (nct * 64 + 8) : 0;
  const int64_t codes = 32 * (ldq + 16);  // aliases the slabs when they are staged (used after them)
  return 2 * 32 * (Kp + 16) + std::max(slab, codes) + 32 * nw * 4 + 32 * 4;
}

// a and b rounded to the layer dtype
template <int DT>
__device__ __forceinline__ void rnd2(float& a, float& b) {
  a = rnd<DT>(a);
  b = rnd<DT>(b);
}

// The out_proj a 32-row output-gate workgroup runs on its own rows' y codes (gate32_kernel with NKO > 0).
struct G32Out {
  const uint8_t* w = nullptr;  // (N, ldw) packed weights, K = N
  int64_t ldw = 0;
  const float* c_w = nullptr;  // per-tensor +1 value
  void* out = nullptr;         // (M, ldo) in the output dtype
  int64_t ldo = 0;
};

// NKO > 0: out_proj (NKO K steps of 32 over y's codes, K = N) follows the gate in the same workgroup.
template <int NW, int NCT, int DT, int NKS, int NKO>
__global__ __launch_bounds__(NW * 64) void gate32_kernel(LinearArgs a, RowQuant o, G32Out op) {
  constexpr int NT = NW * 64;
  constexpr int ARS = G32<NKS>::ARS;
  constexpr int ACH = 2 * 32 * 2 * NKS;        // 16-byte chunks of both operands' activation tiles
  constexpr int AC = (ACH + NT - 1) / NT;
  constexpr int RW = EpRaw<DT, true>::W;
  static_assert(NKS % 4 == 0, "K steps come in 16-byte fragment loads");
  // bf16: each wave stages its own columns of local and gate (32 rows x NCT 32-column tiles) in LDS
  // through row-contiguous 16-byte loads, instead of one 8-byte load per lane and token row
  constexpr bool STG = DT == kBF16;
  constexpr int SP = G32S<NCT>::SP;
  constexpr int SPL = 2 * 32 * NCT * 4 / 64;   // 16-byte slab chunks per lane: 4 per column tile
  extern __shared__ __attribute__((aligned(16))) char lds_g32[];
  char* abuf = lds_g32;                                                  // [2][32][ARS]
  // in-tile indices fit 32 bits: N <= 1024
  const int cp = static_cast<int>(o.ldq) + 16;                           // staged code row pitch
  char* slabs = lds_g32 + 2 * 32 * ARS;                                  // [NW][2][32][SP] (bf16)
  int8_t* codes = reinterpret_cast<int8_t*>(slabs);                      // [32][cp], after the slabs are read
  const int region = STG ? NW * 2 * 32 * SP : 0;
  float* red = reinterpret_cast<float*>(slabs + (region > 32 * cp ? region : 32 * cp));  // [NW][32]
  int32_t* rsl = reinterpret_cast<int32_t*>(red + NW * 32);                            // [32] y code sums
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  __builtin_assume(tid < NT);
  const int h = lane >> 5, row = lane & 31;
  const int N = static_cast<int>(a.N);
  const int col0 = w * NCT * 32;
  const int64_t m0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int64_t m = m0 + row, mc = m < a.M ? m : a.M - 1;  // rows past M compute from row M - 1, never stored

  // 1. every global load first, in straight-line code: packed weight fragments (lane (t, h) of column
  //    tile c: column col0 + 32 c + t, dwords h NKS .. h NKS + NKS - 1), the activation tiles, the row
  //    scales and sums, and the lane's local / gate values
  uint32_t w0[NCT][NKS], w1[NCT][NKS];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    const int n = col0 + 32 * c + row, nc = n < N ? n : N - 1;
    const uint4* p0 = reinterpret_cast<const uint4*>(a.op[0].w + nc * a.op[0].ldw + h * NKS * 4);
    const uint4* p1 = reinterpret_cast<const uint4*>(a.op[1].w + nc * a.op[1].ldw + h * NKS * 4);
#pragma unroll
    for (int i = 0; i < NKS / 4; ++i) {
      const uint4 v0 = p0[i], v1 = p1[i];
      w0[c][4 * i] = v0.x, w0[c][4 * i + 1] = v0.y, w0[c][4 * i + 2] = v0.z, w0[c][4 * i + 3] = v0.w;
      w1[c][4 * i] = v1.x, w1[c][4 * i + 1] = v1.y, w1[c][4 * i + 2] = v1.z, w1[c][4 * i + 3] = v1.w;
    }
  }
  v4i ac[AC];
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    int g = tid + i * NT;
    g = g < ACH ? g : ACH - 1;
    const int p = g / (64 * NKS), rem = g - p * 64 * NKS;
    const int r = rem / (2 * NKS), c = rem - r * 2 * NKS;
    const int64_t mr = m0 + r < a.M ? m0 + r : a.M - 1;
    // operand fields selected by value (a lane-dependent choice of the struct itself would be read
    // from the kernel arguments with a vector load and a full wait)
    const int8_t* q = p == 0 ? a.op[0].q : a.op[1].q;
    const int64_t ldq = p == 0 ? a.op[0].ldq : a.op[1].ldq;
    ac[i] = *reinterpret_cast<const v4i*>(q + mr * ldq + 16 * c);
  }
  // the loads above land first: the products wait for them only, the epilogue's below stay in flight
  __builtin_amdgcn_sched_barrier(0);
  const float sx0 = a.op[0].s_x[mc], sx1 = a.op[1].s_x[mc];
  const int32_t rs0 = a.op[0].rowsum[mc], rs1 = a.op[1].rowsum[mc];
  const float cw0 = a.op[0].c_w[0], cw1 = a.op[1].c_w[0];
  uint32_t lr[NCT][4][RW], gr[NCT][4][RW];
  uint4 sg[STG ? SPL : 1];
  if constexpr (STG) {
    // column tile by column tile (the epilogue of tile c needs only its own chunks): chunk i = 4 c + q
    // of a lane is operand q / 2 (local, gate), row (lane + 64 (q % 2)) / 4, 16-byte chunk lane % 4
#pragma unroll
    for (int i = 0; i < SPL; ++i) {
      const int c = i / 4, q = i % 4;
      const int r = (lane >> 2) + 16 * (q & 1);
      const int64_t mr = m0 + r < a.M ? m0 + r : a.M - 1;
      const int cb = col0 + 32 * c + 8 * (lane & 3);
      const int col = cb < N ? cb : N - 8;  // columns past N: never stored
      if (q < 2)
        sg[i] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.local) + mr * a.ld_local + col);
      else
        sg[i] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.gate) + mr * a.ld_gate + col);
    }
  } else {
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t nb = col0 + 32 * c + 8 * g + 4 * h;
        ep_load<DT, true>(a.local, a.ld_local, mc, nb, a.N, lr[c][g]);
        ep_load<DT, true>(a.gate, a.ld_gate, mc, nb, a.N, gr[c][g]);
      }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. activation tiles into LDS; the code tile's padding columns [N, ldq) are zero
#pragma unroll
  for (int i = 0; i < AC; ++i) {
    const int g = tid + i * NT;
    if (ACH % NT != 0 && g >= ACH) continue;
    const int p = g / (64 * NKS), rem = g - p * 64 * NKS;
    const int r = rem / (2 * NKS), c = rem - r * 2 * NKS;
    *reinterpret_cast<v4i*>(abuf + (p * 32 + r) * ARS + 16 * c) = ac[i];
  }
  // LDS-only barriers throughout: the local / gate loads stay in flight under the products
  lds_barrier();

  // 3. both products: per K step, one B fragment per operand from LDS and NCT weight fragments each
  v16i acc0[NCT], acc1[NCT];
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    acc0[c] = v16i{};
    acc1[c] = v16i{};
  }
  const char* xr0 = abuf + row * ARS + 16 * h * NKS;
  const char* xr1 = abuf + (32 + row) * ARS + 16 * h * NKS;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) {
    const v4i x0 = *reinterpret_cast<const v4i*>(xr0 + 16 * ks);
    const v4i x1 = *reinterpret_cast<const v4i*>(xr1 + 16 * ks);
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      acc0[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(unpack_frag(w0[c][ks]), x0, acc0[c], 0, 0, 0);
      acc1[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(unpack_frag(w1[c][ks]), x1, acc1[c], 0, 0, 0);
    }
  }

  // out_proj's weight fragments (same lane assignment as the gate's: column col0 + 32 c + t, dwords
  // h NKO .. h NKO + NKO - 1): requested now, they land under the gate's epilogue arithmetic
  uint32_t w2[NKO > 0 ? NCT : 1][NKO > 0 ? NKO : 1];
  if constexpr (NKO > 0) {
#pragma unroll
    for (int c = 0; c < NCT; ++c) {
      const int n = col0 + 32 * c + row, nc = n < N ? n : N - 1;
      const uint4* p2 = reinterpret_cast<const uint4*>(op.w + nc * op.ldw + h * NKO * 4);
#pragma unroll
      for (int i = 0; i < NKO / 4; ++i) {
        const uint4 v = p2[i];
        w2[c][4 * i] = v.x, w2[c][4 * i + 1] = v.y, w2[c][4 * i + 2] = v.z, w2[c][4 * i + 3] = v.w;
      }
    }
  }

  // the wave's local / gate slab into its own LDS region (read back by the same wave only: LDS
  // operations of one wave complete in order, the wave barrier keeps the compiler from moving them)
  char* slab = slabs + w * 2 * 32 * SP;

  // 4. y = local + sigmoid(gate) * state_proj + ent_proj in the reference's op order (tesm.py:1256-1260),
  //    every op rounded to the layer dtype; columns past N are 0
  const float inv0 = 1.0f / sx0, inv1 = 1.0f / sx1;
  float y[NCT][16];
  float mx = 0.0f;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    if (col0 + 32 * c >= N) continue;  // N % 32 == 0: a column tile is all in range or all out (uniform)
    if constexpr (STG) {
      // this tile's local / gate chunks into the wave's own LDS slab, read back by the same wave only
      // (LDS operations of one wave complete in order; the wave barriers keep the compiler from moving them)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = (lane >> 2) + 16 * (q & 1);
        uint2* d = reinterpret_cast<uint2*>(slab + ((q >> 1) * 32 + r) * SP + 64 * c + 16 * (lane & 3));
        d[0] = make_uint2(sg[4 * c + q].x, sg[4 * c + q].y);
        d[1] = make_uint2(sg[4 * c + q].z, sg[4 * c + q].w);
      }
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if constexpr (STG) {
        const int off = (32 * c + 8 * g + 4 * h) * 2;
        const uint2 l2 = *reinterpret_cast<const uint2*>(slab + row * SP + off);
        const uint2 g2 = *reinterpret_cast<const uint2*>(slab + (32 + row) * SP + off);
        lr[c][g][0] = l2.x, lr[c][g][1] = l2.y, gr[c][g][0] = g2.x, gr[c][g][1] = g2.y;
      }
      float sp[4], ep[4], gv[4], v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        // (acc / s_x) * c_w as the tiled kernels form it, so that every output-gate kernel agrees bit for bit
        sp[r] = (static_cast<float>(acc0[c][4 * g + r] - rs0) * inv0) * cw0;
        ep[r] = (static_cast<float>(acc1[c][4 * g + r] - rs1) * inv1) * cw1;
        gv[r] = sigmoidf_(ep_get<DT, true>(gr[c][g], r));
      }
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        rnd2<DT>(sp[r], sp[r + 1]);
        rnd2<DT>(ep[r], ep[r + 1]);
        rnd2<DT>(gv[r], gv[r + 1]);
        v[r] = gv[r] * sp[r];
        v[r + 1] = gv[r + 1] * sp[r + 1];
        rnd2<DT>(v[r], v[r + 1]);
        v[r] = ep_get<DT, true>(lr[c][g], r) + v[r];
        v[r + 1] = ep_get<DT, true>(lr[c][g], r + 1) + v[r + 1];
        rnd2<DT>(v[r], v[r + 1]);
        v[r] = v[r] + ep[r];
        v[r + 1] = v[r + 1] + ep[r + 1];
        rnd2<DT>(v[r], v[r + 1]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        y[c][4 * g + r] = v[r];
        mx = fmaxf(mx, fabsf(v[r]));
      }
    }
  }
  if (o.y && m < a.M) {  // the optional y itself (decision taps)
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nb = col0 + 32 * c + 8 * g + 4 * h;
        if (nb < N) {
          const float yy[4] = {y[c][4 * g], y[c][4 * g + 1], y[c][4 * g + 2], y[c][4 * g + 3]};
          store4<DT>(o.y, m * o.ldy + nb, yy, vec4_ok<DT>(o.y, o.ldy));
        }
      }
  }

  // 5. per-token absmax over the workgroup's columns, then int8 codes into LDS in layout 1: column
  //    n = 16 G + e sits at byte 16 G + 4 (e & 3) + (e >> 2); here e = 8 (g & 1) + 4 h + r
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  if (h == 0) red[w * 32 + row] = mx;
  lds_barrier();  // every wave is past its slab reads: the code tile may overwrite them
  const int padw = (static_cast<int>(o.ldq) - N) / 4;  // N % 32 == 0, ldq % 16 == 0
  if (padw > 0)
    for (int i = tid; i < 32 * padw; i += NT)
      reinterpret_cast<uint32_t*>(codes + (i / padw) * cp + N)[i % padw] = 0u;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < NW; ++i) amax = fmaxf(amax, red[i * 32 + row]);
  const float sc = act_scale<DT>(amax, o.eps);
  int8_t* crow = codes + row * cp + col0 + h;
#pragma unroll
  for (int c = 0; c < NCT; ++c) {
    if (col0 + 32 * c >= N) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float t[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) t[r] = y[c][4 * g + r] * sc;
      rnd2<DT>(t[0], t[1]);
      rnd2<DT>(t[2], t[3]);
#pragma unroll
      for (int r = 0; r < 4; ++r)  // clamp, then + 1.5 * 2^23 rounds to the code, left in the low byte (group_codes)
        reinterpret_cast<uint8_t*>(crow)[32 * c + 16 * (g >> 1) + 4 * r + 2 * (g & 1)] =
            static_cast<uint8_t>(__float_as_uint(fminf(fmaxf(t[r], -128.0f), 127.0f) + 12582912.0f));
    }
  }
  lds_barrier();

  // 6. the code tile out, row by row in 16-byte chunks; each row's code sum by v_dot4 over its chunks
  constexpr int TPR = NT / 32;  // threads per row
  const int r = tid / TPR, tr = tid % TPR;
  const int chunks = static_cast<int>(o.ldq / 16);
  const int64_t mr = m0 + r;
  int sum = 0;
  for (int ck = tr; ck < chunks; ck += TPR) {
    const uint4 v = *reinterpret_cast<const uint4*>(codes + r * cp + 16 * ck);
    sum = __builtin_amdgcn_sdot4(static_cast<int>(v.x), 0x01010101, sum, false);
    sum = __builtin_amdgcn_sdot4(static_cast<int>(v.y), 0x01010101, sum, false);
    sum = __builtin_amdgcn_sdot4(static_cast<int>(v.z), 0x01010101, sum, false);
    sum = __builtin_amdgcn_sdot4(static_cast<int>(v.w), 0x01010101, sum, false);
    if (o.q && mr < a.M) reinterpret_cast<uint4*>(o.q + mr * o.ldq)[ck] = v;
  }
  sum = wave_sum_i<TPR>(sum);  // the row's TPR consecutive lanes; DPP steps, an integer sum in any order
  if (tr == 0 && o.q && mr < a.M) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < NW; ++i) am = fmaxf(am, red[i * 32 + r]);
    o.s[mr] = act_scale<DT>(am, o.eps);
    o.rs[mr] = sum;
  }
  if constexpr (NKO > 0) {
    if (tr == 0) rsl[r] = sum;
    lds_barrier();
    // 7. out_proj on the workgroup's y codes (the B operand from the code tile, K split between the lane
    //    halves as the gate's products split it), then its plain epilogue (acc - rowsum) / s_x * c_w, the
    //    tiled kernels' op order, so the result equals a separate out_proj bit for bit
    v16i acc2[NCT];
#pragma unroll
    for (int c = 0; c < NCT; ++c) acc2[c] = v16i{};
    const char* xr = reinterpret_cast<const char*>(codes) + row * cp + 16 * h * NKO;
#pragma unroll
    for (int ks = 0; ks < NKO; ++ks) {
      const v4i x = *reinterpret_cast<const v4i*>(xr + 16 * ks);
#pragma unroll
      for (int c = 0; c < NCT; ++c)
        acc2[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(unpack_frag(w2[c][ks]), x, acc2[c], 0, 0, 0);
    }
    const int32_t rsy = rsl[row];
    const float invy = 1.0f / sc, cwo = op.c_w[0];
    if (DT == kBF16 && reinterpret_cast<uintptr_t>(op.out) % 16 == 0 && op.ldo % 8 == 0) {
      // staged through the wave's own 32 x 80-byte LDS slab, one column tile at a time, so that a store
      // instruction covers 16 rows x 64 contiguous bytes instead of 32 rows x 8
      char* os = reinterpret_cast<char*>(rsl + 32) + w * 32 * 80;
#pragma unroll
      for (int c = 0; c < NCT; ++c) {
        if (col0 + 32 * c >= N) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) v[rr] = (static_cast<float>(acc2[c][4 * g + rr] - rsy) * invy) * cwo;
          *reinterpret_cast<uint2*>(os + row * 80 + (8 * g + 4 * h) * 2) =
              make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          const int idx = 64 * it + lane, rr = idx >> 2, ch = idx & 3;
          const uint4 d = *reinterpret_cast<const uint4*>(os + rr * 80 + 16 * ch);
          if (m0 + rr < a.M)
            *reinterpret_cast<uint4*>(static_cast<uint16_t*>(op.out) + (m0 + rr) * op.ldo + col0 + 32 * c + 8 * ch) = d;
        }
        __builtin_amdgcn_wave_barrier();
      }
      return;
    }
    if (m >= a.M) return;
    const bool vo = vec4_ok<DT>(op.out, op.ldo);
#pragma unroll
    for (int c = 0; c < NCT; ++c)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int nb = col0 + 32 * c + 8 * g + 4 * h;
        if (nb >= N) continue;
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) v[rr] = (static_cast<float>(acc2[c][4 * g + rr] - rsy) * invy) * cwo;
        store4<DT>(op.out, m * op.ldo + nb, v, vo);
      }
  }
}

template <int WM, int WN, int TM, int TN, int EPI, int NS = 0>
int run_mfma32(const LinearArgs& a, hipStream_t st) {
  using C = Cfg32<WM, WN, TM, TN>;
  const int64_t tiles = ((a.N + C::BN - 1) / C::BN) * ((a.M + C::BM - 1) / C::BM);
  TESM_REQUIRE(tiles <= 0x7fffffff, kErrUnsupported, "bitlinear: too many tiles");
  const unsigned grid = static_cast<unsigned>(tiles);
  if (a.out_dt == kBF16)
    mfma32_kernel<WM, WN, TM, TN, EPI, kBF16, NS><<<grid, C::NT, 0, TESM_LOGGED(st, mfma32_kernel<WM, WN, TM, TN, EPI, kBF16, NS>)>>>(a);
  else
    mfma32_kernel<WM, WN, TM, TN, EPI, kF32, NS><<<grid, C::NT, 0, TESM_LOGGED(st, mfma32_kernel<WM, WN, TM, TN, EPI, kF32, NS>)>>>(a);
  return check_launch("bitlinear mfma32");
}

struct DeviceLimits {
  int cus = 0;
  int64_t lds = 0;
};

// Compute units and LDS bytes per workgroup of the current device (queried once per device).
inline DeviceLimits device_limits() {
  static DeviceLimits cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DeviceLimits{};
  DeviceLimits& d = cache[dev];
  if (d.cus == 0) {
    int cus = 0, lds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
      return DeviceLimits{};
    d.lds = lds;
    d.cus = cus;
  }
  return d;
}

template <int NW, int TM, int TN, int EPI>
int run_skinny(const LinearArgs& a, hipStream_t st) {
  const int64_t tiles = ((a.M + 16 * TM - 1) / (16 * TM)) * ((a.N + 16 * TN - 1) / (16 * TN));
  TESM_REQUIRE(tiles <= 0x7fffffff, kErrUnsupported, "bitlinear: too many tiles");
  if (a.out_dt == kBF16)
    skinny_kernel<NW, TM, TN, EPI, kBF16><<<static_cast<unsigned>(tiles), NW * 64, 0, TESM_LOGGED(st, skinny_kernel<NW, TM, TN, EPI, kBF16>)>>>(a);
  else
    skinny_kernel<NW, TM, TN, EPI, kF32><<<static_cast<unsigned>(tiles), NW * 64, 0, TESM_LOGGED(st, skinny_kernel<NW, TM, TN, EPI, kF32>)>>>(a);
  return check_launch("bitlinear skinny");
}

template <int WM, int WN, int TM, int TN, int EPI>
int run_mfma(const LinearArgs& a, hipStream_t st) {
  using C = Cfg<WM, WN, TM, TN>;
  const int64_t tiles = ((a.N + C::BN - 1) / C::BN) * ((a.M + C::BM - 1) / C::BM);
  TESM_REQUIRE(tiles <= 0x7fffffff, kErrUnsupported, "bitlinear: too many tiles");
  const unsigned grid = static_cast<unsigned>(tiles);
  if (a.out_dt == kBF16)
    mfma_kernel<WM, WN, TM, TN, EPI, kBF16><<<grid, C::NT, 0, TESM_LOGGED(st, mfma_kernel<WM, WN, TM, TN, EPI, kBF16>)>>>(a);
  else
    mfma_kernel<WM, WN, TM, TN, EPI, kF32><<<grid, C::NT, 0, TESM_LOGGED(st, mfma_kernel<WM, WN, TM, TN, EPI, kF32>)>>>(a);
  return check_launch("bitlinear mfma");
}

inline bool host_vec4_ok(const void* p, int64_t ld, int dt) {
  const int64_t bytes = dt == kBF16 ? 8 : 16;
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0 && (ld * (dt == kBF16 ? 2 : 4)) % bytes == 0;
}

template <int NW, int NCT, int NKS>
void launch_rowq_lds(const LinearArgs& a, const RowQuant& o, int64_t ntiles, int64_t lds, int cus, hipStream_t st) {
  // register-resident weights: one workgroup per CU (VGPR-bound), its tiles prefetched one ahead
  const int64_t per_cu = rowq_reg_weights<NKS>() ? 1 : std::max<int64_t>(1, std::min<int64_t>(4, (160 * 1024) / lds));
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>(ntiles, cus * per_cu));
  if (a.out_dt == kBF16)
    gate_rowq_lds_kernel<NW, NCT, kBF16, NKS><<<grid, NW * 64, lds, TESM_LOGGED(st, gate_rowq_lds_kernel<NW, NCT, kBF16, NKS>)>>>(a, o, ntiles);
  else
    gate_rowq_lds_kernel<NW, NCT, kF32, NKS><<<grid, NW * 64, lds, TESM_LOGGED(st, gate_rowq_lds_kernel<NW, NCT, kF32, NKS>)>>>(a, o, ntiles);
}

template <int NW, int NCT>
int run_rowq(const LinearArgs& a, const RowQuant& o, hipStream_t st) {
  const bool per_row = a.op[0].c_w_per_row || a.op[1].c_w_per_row;
  const int64_t ntiles = (a.M + 15) / 16;
  const bool vec = a.N % 4 == 0 && host_vec4_ok(a.local, a.ld_local, a.out_dt) &&
                   host_vec4_ok(a.gate, a.ld_gate, a.out_dt);
  const int64_t nks = a.Kp / 64;
  if (vec && (nks == 2 || nks == 4 || nks == 8)) {
    const DeviceLimits dl = device_limits();
    const int64_t lds = rowq_lds_bytes(a.N, nks, o.ldq, NW);
    if (dl.cus > 0 && lds <= dl.lds) {
      if (nks == 2)
        launch_rowq_lds<NW, NCT, 2>(a, o, ntiles, lds, dl.cus, st);
      else if (nks == 4)
        launch_rowq_lds<NW, NCT, 4>(a, o, ntiles, lds, dl.cus, st);
      else
        launch_rowq_lds<NW, NCT, 8>(a, o, ntiles, lds, dl.cus, st);
      return check_launch("output gate rowq (LDS weights)");
    }
  }
  const size_t lds = static_cast<size_t>(16 * o.ldq + 2 * 16 * NW * 4 + (per_row ? 2 * a.N * 4 : 0));
  const unsigned grid = static_cast<unsigned>(ntiles);
  if (a.out_dt == kBF16) {
    if (vec)
      gate_rowq_kernel<NW, NCT, kBF16, true, 0><<<grid, NW * 64, lds, TESM_LOGGED(st, gate_rowq_kernel<NW, NCT, kBF16, true, 0>)>>>(a, o);
    else
      gate_rowq_kernel<NW, NCT, kBF16, false, 0><<<grid, NW * 64, lds, TESM_LOGGED(st, gate_rowq_kernel<NW, NCT, kBF16, false, 0>)>>>(a, o);
  } else {
    if (vec)
      gate_rowq_kernel<NW, NCT, kF32, true, 0><<<grid, NW * 64, lds, TESM_LOGGED(st, gate_rowq_kernel<NW, NCT, kF32, true, 0>)>>>(a, o);
    else
      gate_rowq_kernel<NW, NCT, kF32, false, 0><<<grid, NW * 64, lds, TESM_LOGGED(st, gate_rowq_kernel<NW, NCT, kF32, false, 0>)>>>(a, o);
  }
  return check_launch("output gate rowq");
}

template <int NW, int NCT, int NKS, int NKO = 0>
void launch_gate32(const LinearArgs& a, const RowQuant& o, int64_t lds, hipStream_t st, const G32Out& op = G32Out{}) {
  const unsigned grid = static_cast<unsigned>((a.M + 31) / 32);
  if (a.out_dt == kBF16)
    gate32_kernel<NW, NCT, kBF16, NKS, NKO><<<grid, NW * 64, lds, TESM_LOGGED(st, gate32_kernel<NW, NCT, kBF16, NKS, NKO>)>>>(a, o, op);
  else if constexpr (NKO == 0)  // the fused out_proj is bf16 only (in float32 its registers would spill)
    gate32_kernel<NW, NCT, kF32, NKS, NKO><<<grid, NW * 64, lds, TESM_LOGGED(st, gate32_kernel<NW, NCT, kF32, NKS, NKO>)>>>(a, o, op);
}

template <int NCT>
void launch_gate32_k(const LinearArgs& a, const RowQuant& o, int64_t nks, int64_t lds, hipStream_t st) {
  if (nks == 4)
    launch_gate32<8, NCT, 4>(a, o, lds, st);
  else if (nks == 8)
    launch_gate32<8, NCT, 8>(a, o, lds, st);
  else
    launch_gate32<8, NCT, 12>(a, o, lds, st);
}

// The 32-row kernel when it applies: per-tensor weight scales, N a multiple of 32 up to 1024, K up to
// 384 (register-resident weights), vector-aligned local / gate rows and an LDS budget that fits.
int try_gate32(const LinearArgs& a, const RowQuant& o, hipStream_t st) {
  // TESM_HIP_NO_GATE32=1 keeps the 16-row kernel (a diagnostic switch for side-by-side timing)
  static const bool off = [] {
    const char* e = std::getenv("TESM_HIP_NO_GATE32");
    return e != nullptr && e[0] == '1';
  }();
  const int64_t nks = a.Kp / 32;
  if (off) return -1;
  // bf16 slabs are read in 16-byte chunks: rows and bases 16-byte aligned
  const bool a16 = a.out_dt != kBF16 || (reinterpret_cast<uintptr_t>(a.local) % 16 == 0 && a.ld_local % 8 == 0 &&
                                        reinterpret_cast<uintptr_t>(a.gate) % 16 == 0 && a.ld_gate % 8 == 0);
  if (a.op[0].c_w_per_row || a.op[1].c_w_per_row || a.N % 32 != 0 || a.N > 1024 ||
      !(nks == 4 || nks == 8 || nks == 12) || !host_vec4_ok(a.local, a.ld_local, a.out_dt) ||
      !host_vec4_ok(a.gate, a.ld_gate, a.out_dt) || !a16 || (o.y && !host_vec4_ok(o.y, o.ldy, a.out_dt)))
    return -1;
  const DeviceLimits dl = device_limits();
  const int64_t nct = (a.N / 32 + 7) / 8;
  const int64_t lds = gate32_lds_bytes(a.Kp, o.ldq, nct, 8, a.out_dt == kBF16);
  if (dl.cus <= 0 || lds > dl.lds) return -1;
  if (nct == 1)
    launch_gate32_k<1>(a, o, nks, lds, st);
  else if (nct == 2)
    launch_gate32_k<2>(a, o, nks, lds, st);
  else if (nct == 3)
    launch_gate32_k<3>(a, o, nks, lds, st);
  else
    launch_gate32_k<4>(a, o, nks, lds, st);
  return check_launch("output gate (32-row tiles)");
}

template <int LPR, int MR, int NCH, int RPG = 4>
int run_gemv(const LinearArgs& a, hipStream_t st) {
  constexpr int GPW = 64 / LPR;
  const int64_t groups = (a.N + RPG - 1) / RPG;
  const int64_t waves = (groups + GPW - 1) / GPW;
  const unsigned blocks = static_cast<unsigned>((waves + 3) / 4);
  if (a.out_dt == kBF16)
    gemv_kernel<LPR, MR, NCH, kBF16, RPG><<<blocks, 256, 0, TESM_LOGGED(st, gemv_kernel<LPR, MR, NCH, kBF16, RPG>)>>>(a);
  else
    gemv_kernel<LPR, MR, NCH, kF32, RPG><<<blocks, 256, 0, TESM_LOGGED(st, gemv_kernel<LPR, MR, NCH, kF32, RPG>)>>>(a);
  return check_launch("bitlinear gemv");
}

template <int MR>
int dispatch_gemv(const LinearArgs& a, int64_t nch, hipStream_t st) {
  if (nch <= 4) return run_gemv<4, MR, 1>(a, st);
  if (nch <= 8) return run_gemv<8, MR, 1>(a, st);
  if (nch <= 16) return run_gemv<16, MR, 1>(a, st);
  if (nch <= 32) return run_gemv<32, MR, 1>(a, st);
  // two rows per lane group: twice the waves of four, 3-7 % faster at K = 4096 (N 4096 / 11008)
  if (nch <= 64) return run_gemv<64, MR, 1, 2>(a, st);
  if (nch <= 128) return run_gemv<64, MR, 2, 2>(a, st);
  return run_gemv<64, MR, 4, 2>(a, st);
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

// Two-product epilogues: split-K for decode-size batches, else the 32x32 kernels as for plain products.
template <int EPI>
int dispatch_dual(const LinearArgs& a, hipStream_t st) {
  if (a.M <= 16) return run_skinny<4, 1, 1, EPI>(a, st);
  if (a.M <= 32) return run_skinny<4, 2, 1, EPI>(a, st);
  const int64_t tiles256 = ((a.M + 127) / 128) * ((a.N + 255) / 256);
  // long K on many tiles (the MIMO output gate, K 2 x 8192): two direct-to-LDS stages, 694 us vs 766 us
  // with three at M 8192
  if (a.N % 256 == 0 && tiles256 >= 2048 && a.Kp >= 2048) return run_mfma32<2, 4, 2, 2, EPI, 2>(a, st);
  if (a.N % 256 == 0 && tiles256 >= 128) return run_mfma32<2, 4, 2, 2, EPI>(a, st);
  return run_mfma32<1, 4, 2, 1, EPI>(a, st);
}

// Waves of a fused-quantization workgroup (16 waves, four per SIMD, were measured no faster at the
// decode shapes: the quantization phase is bound by its dependent load / reduction / LDS steps).
constexpr int kFqNW = 4;

// LDS of one fused-quantization workgroup: 16 TM code rows of Kp + 16 bytes with their scales and sums
// (dynamic), and skinny_body's static split-K reduction buffer (kFqNW - 1 waves' TM partial tiles, 16
// bytes per lane each).
static int64_t linear_fq_lds_bytes(int64_t M, int64_t Kp) {
  const int64_t TM = M <= 16 ? 1 : 2;
  return 16 * TM * (Kp + 16) + 16 * TM * 8 + (kFqNW - 1) * TM * 64 * 16;
}

// Kp <= 1920 keeps a workgroup at most 68 KB of LDS; the device's per-workgroup limit is checked too (a
// build for a target with less LDS takes the two-launch path).
bool linear_fq_ok(const LinearArgs& a) {
  if (!(a.epilogue == kEpiStore && a.M > 4 && a.M <= 32 && a.N >= 1 && a.N < 16384 && a.Kp >= kKTile &&
        a.Kp % kKTile == 0 && a.Kp <= 1920))
    return false;
  const DeviceLimits dl = device_limits();
  return dl.lds > 0 && linear_fq_lds_bytes(a.M, a.Kp) <= dl.lds;
}

namespace {
template <int TM, int DT, bool VEC, int G>
void run_skinny_fq(const LinearArgs& a, const FusedQuantIn& f, hipStream_t st) {
  const int64_t tiles = ((a.M + 16 * TM - 1) / (16 * TM)) * ((a.N + 15) / 16);
  const size_t lds = static_cast<size_t>(16 * TM * (a.Kp + 16) + 16 * TM * 8);
  if (a.out_dt == kBF16)
    skinny_fq_kernel<kFqNW, TM, 1, kBF16, DT, VEC, G><<<static_cast<unsigned>(tiles), kFqNW * 64, lds, TESM_LOGGED(st, skinny_fq_kernel<kFqNW, TM, 1, kBF16, DT, VEC, G>)>>>(a, f);
  else
    skinny_fq_kernel<kFqNW, TM, 1, kF32, DT, VEC, G><<<static_cast<unsigned>(tiles), kFqNW * 64, lds, TESM_LOGGED(st, skinny_fq_kernel<kFqNW, TM, 1, kF32, DT, VEC, G>)>>>(a, f);
}
template <int TM>
void dispatch_skinny_fq(const LinearArgs& a, const FusedQuantIn& f, bool vec, hipStream_t st) {
  // groups per lane: Kp / 16 over kFqNW * 64 / (16 TM) lanes per row; the register-held variants (one read
  // of the row, straight-line loads) need 16-byte aligned rows of whole 16-element groups
  const int64_t lpr = kFqNW * 64 / (16 * TM), gpl = (a.Kp / 16 + lpr - 1) / lpr;
  const bool held = vec && f.K % 16 == 0;
  if (f.dt == kBF16) {
    if (held) {
      if (gpl <= 2) return run_skinny_fq<TM, kBF16, true, 2>(a, f, st);
      if (gpl <= 4) return run_skinny_fq<TM, kBF16, true, 4>(a, f, st);
      if (gpl <= 6) return run_skinny_fq<TM, kBF16, true, 6>(a, f, st);
      if (gpl <= 8) return run_skinny_fq<TM, kBF16, true, 8>(a, f, st);
    }
    if (vec) return run_skinny_fq<TM, kBF16, true, 0>(a, f, st);
    return run_skinny_fq<TM, kBF16, false, 0>(a, f, st);
  }
  if (held) {
    if (gpl <= 2) return run_skinny_fq<TM, kF32, true, 2>(a, f, st);
    if (gpl <= 4) return run_skinny_fq<TM, kF32, true, 4>(a, f, st);
  }
  if (vec) return run_skinny_fq<TM, kF32, true, 0>(a, f, st);
  return run_skinny_fq<TM, kF32, false, 0>(a, f, st);
}
}  // namespace

int launch_linear_fq(const LinearArgs& a, const FusedQuantIn& f, hipStream_t st) {
  TESM_REQUIRE(linear_fq_ok(a), kErrUnsupported, "bitlinear fused quant: needs 4 < M <= 32, N < 16384, Kp <= 1920");
  TESM_REQUIRE(f.dt == kF32 || f.dt == kBF16, kErrInvalidArg, "bitlinear fused quant: x dtype must be 0 or 1");
  TESM_REQUIRE(f.x && f.K >= 1 && f.K <= a.Kp && f.ldx >= f.K, kErrInvalidArg, "bitlinear fused quant: bad x");
  TESM_REQUIRE(a.out_dt == kF32 || a.out_dt == kBF16, kErrInvalidArg, "bitlinear: out dtype must be 0 or 1");
  TESM_REQUIRE(a.out && a.ldo >= a.N, kErrInvalidArg, "bitlinear: need out and ldo >= N");
  const LinearOperand& o = a.op[0];
  TESM_REQUIRE(o.w && o.c_w && o.ldw >= a.Kp / 4 && o.ldw % 16 == 0 && aligned(o.w, 16), kErrInvalidArg,
               "bitlinear fused quant: bad packed weights");
  const int esz = f.dt == kBF16 ? 2 : 4;
  const bool vec = aligned(f.x, 16) && (f.ldx * esz) % 16 == 0;
  if (a.M <= 16)
    dispatch_skinny_fq<1>(a, f, vec, st);
  else
    dispatch_skinny_fq<2>(a, f, vec, st);
  return check_launch("bitlinear skinny (fused quant)");
}

// Store-epilogue products of more than 32 rows on the 32x32x32 MFMA kernels (EPI kEpiStore or
// kEpiGates).
template <int EPI>
int dispatch_store32(const LinearArgs& a, hipStream_t st) {
  // 32x32x32 MFMA kernels: 128x256 tiles (8 waves of 64x64) when N fills them and there are
  // enough of them, 128x128 (4 waves of 64x64) when those still give two workgroups per CU,
  // else 64x128 (4 waves side by side along N); measured at the layer shapes (in_proj /
  // out_proj / configs[1] / configs[4])
  const int64_t tiles256 = ((a.M + 127) / 128) * ((a.N + 255) / 256);
  const int64_t tiles128 = ((a.M + 127) / 128) * ((a.N + 127) / 128);
  // long K loops over many tiles: direct-to-LDS loads into two stages (no staging registers);
  // MIMO in_proj at M 8192: 1048 us vs 1069 us with three stages
  if (a.N % 256 == 0 && tiles256 >= 2048 && a.Kp >= 2048) return run_mfma32<2, 4, 2, 2, EPI, 2>(a, st);
  // short K on a few hundred 128x256 tiles (the SISO in_proj: 8192 x 2432 x 768; the LM head: 512 x
  // 151936 x 768): two direct-to-LDS stages (48 KB; registers allow two workgroups per CU either
  // way): 23.6 us vs 25.6 us with three stages and 27.6 us for register-staged 128x128 tiles; LM
  // head 74 us vs 82 us
  if (tiles256 >= 512 && a.Kp <= 1024) {
    // more 128x256 tiles than two rounds of the CUs with a narrow remainder (the SISO in_proj: 640
    // tiles): the columns past two tiles per CU go to 128x128 tiles (the split kernel)
    const int cus = device_limits().cus;
    const int64_t ntm = (a.M + 127) / 128;
    const int64_t ntnA = cus > 0 ? std::min<int64_t>(a.N / 256, (2 * cus) / ntm) : 0;
    const int64_t nA = ntnA * 256;
    constexpr int TMB = 2;  // 128-row tail tiles (64-row ones: 26.7 against 26.1 us in the layer)
    const int64_t ntmB = (a.M + 64 * TMB - 1) / (64 * TMB), ntnB = (a.N - nA + 127) / 128;
    if (ntnA >= 1 && a.N > nA && a.N - nA <= 512 && ntm * ntnA + ntmB * ntnB <= 0x7fffffff) {
      const unsigned grid = static_cast<unsigned>(ntm * ntnA + ntmB * ntnB);
      if (a.out_dt == kBF16)
        mfma32_split_kernel<kBF16, TMB, EPI><<<grid, 512, 0, TESM_LOGGED(st, mfma32_split_kernel<kBF16, TMB, EPI>)>>>(a, nA);
      else
        mfma32_split_kernel<kF32, TMB, EPI><<<grid, 512, 0, TESM_LOGGED(st, mfma32_split_kernel<kF32, TMB, EPI>)>>>(a, nA);
      return check_launch("bitlinear mfma32 split");
    }
    return run_mfma32<2, 4, 2, 2, EPI, 2>(a, st);
  }
  // fewer 128x256 tiles than CUs at short K (the SISO out_proj: 8192 x 768 x 768): 64x128 tiles, two
  // direct-to-LDS stages: 10.1 us vs 10.7 us for 128x256 tiles
  if (tiles256 < 256 && a.Kp <= 1024) return run_mfma32<1, 4, 2, 1, EPI, 2>(a, st);
  if (a.N % 256 == 0 && tiles256 >= 128) return run_mfma32<2, 4, 2, 2, EPI>(a, st);
  if (tiles128 >= 512) return run_mfma32<2, 2, 2, 2, EPI>(a, st);
  return run_mfma32<1, 4, 2, 1, EPI>(a, st);
}

int launch_linear(const LinearArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.M >= 0 && a.N >= 0, kErrInvalidArg, "bitlinear: negative size");
  TESM_REQUIRE(a.Kp >= kKTile && a.Kp % kKTile == 0, kErrInvalidArg, "bitlinear: Kp must be a positive multiple of 128");
  TESM_REQUIRE(a.out_dt == kF32 || a.out_dt == kBF16, kErrInvalidArg, "bitlinear: out dtype must be 0 or 1");
  TESM_REQUIRE(a.epilogue == kEpiStore || a.epilogue == kEpiOutputGate || a.epilogue == kEpiSwiGLU ||
                   a.epilogue == kEpiGates,
               kErrInvalidArg, "bitlinear: bad epilogue");
  if (a.M == 0 || a.N == 0) return kOk;
  TESM_REQUIRE(a.out && a.ldo >= a.N, kErrInvalidArg, "bitlinear: need out and ldo >= N");
  if (int rc = check_operand(a.op[0], a.Kp, "op0")) return rc;
  if (a.epilogue == kEpiGates) {
    TESM_REQUIRE(a.M > 32 && !a.bias && !a.acc_dump && !a.op[0].c_w_per_row && a.act_bias && a.act_w > 0 &&
                     a.act_n0 >= 0 && a.act_n0 % 32 == 0 && a.act_w % 32 == 0 && a.act_n0 + 3 * a.act_w <= a.N,
                 kErrUnsupported, "bitlinear gates epilogue: needs M > 32, 32-aligned regions inside N, no bias");
    return dispatch_store32<kEpiGates>(a, st);
  }
  if (a.epilogue != kEpiStore) {
    if (int rc = check_operand(a.op[1], a.Kp, "op1")) return rc;
    TESM_REQUIRE(a.bias == nullptr, kErrInvalidArg, "bitlinear two-product epilogue: bias unsupported");
  }
  if (a.epilogue == kEpiOutputGate)
    TESM_REQUIRE(a.local && a.gate && a.ld_local >= a.N && a.ld_gate >= a.N, kErrInvalidArg,
                 "bitlinear output gate: need local and gate operands");
  const int64_t nch = a.Kp / 64;
  if (a.epilogue == kEpiStore && a.M <= 4 && nch <= 256) {
    if (a.M == 1) return dispatch_gemv<1>(a, nch, st);
    if (a.M == 2) return dispatch_gemv<2>(a, nch, st);
    return dispatch_gemv<4>(a, nch, st);
  }
  if (a.epilogue == kEpiStore) {
    // decode-size batches: the split-K kernel while the LDS-staged one would have too few 64-column
    // tiles to fill the chip (measured at M = 32: N = 768 .. 4096 faster split, N = 34816 staged)
    if (a.M <= 16 && a.N < 16384) return run_skinny<4, 1, 1, kEpiStore>(a, st);
    if (a.M <= 32 && a.N < 16384) return run_skinny<4, 2, 1, kEpiStore>(a, st);
    // decode-size batches over wide weights (MIMO decode in_proj, 32 x 34816 x 4096): 32x128 tiles on
    // the 32x32x32 form, 16.5 us vs 19.3 us for 32x64 tiles on the 16x16x64 one
    if (a.M <= 32) return run_mfma32<1, 4, 1, 1, kEpiStore>(a, st);
    return dispatch_store32<kEpiStore>(a, st);
  }
  if (a.epilogue == kEpiOutputGate) return dispatch_dual<kEpiOutputGate>(a, st);
  return dispatch_dual<kEpiSwiGLU>(a, st);
}

int launch_gate_out(const LinearArgs& a, const RowQuant& o, const LinearOperand& out_proj, void* out, int64_t ldout,
                    hipStream_t st) {
  static const bool off = [] {
    const char* e = std::getenv("TESM_HIP_NO_GATE32");
    return e != nullptr && e[0] == '1';
  }();
  if (off || a.epilogue != kEpiOutputGate || a.M <= 0 || a.N != 768 || a.out_dt != kBF16) return -1;
  const int64_t nks = a.Kp / 32;
  // out_proj over y's codes: K = N = 768 (24 K steps), per-tensor scale, rows of the code pitch
  if (!out_proj.w || !out_proj.c_w || out_proj.c_w_per_row || o.ldq != kpad(a.N) || out_proj.ldw * 4 != o.ldq ||
      !aligned(out_proj.w, 16) || !out || ldout < a.N)
    return -1;
  if (o.q && !(o.s && o.rs && o.ldq % 16 == 0 && aligned(o.q, 16))) return -1;
  const bool a16 = a.out_dt != kBF16 || (reinterpret_cast<uintptr_t>(a.local) % 16 == 0 && a.ld_local % 8 == 0 &&
                                        reinterpret_cast<uintptr_t>(a.gate) % 16 == 0 && a.ld_gate % 8 == 0);
  if (a.op[0].c_w_per_row || a.op[1].c_w_per_row || !(nks == 4 || nks == 8 || nks == 12) ||
      !host_vec4_ok(a.local, a.ld_local, a.out_dt) || !host_vec4_ok(a.gate, a.ld_gate, a.out_dt) || !a16 ||
      (o.y && !host_vec4_ok(o.y, o.ldy, a.out_dt)))
    return -1;
  if (int rc = check_operand(a.op[0], a.Kp, "op0")) return rc;
  if (int rc = check_operand(a.op[1], a.Kp, "op1")) return rc;
  const DeviceLimits dl = device_limits();
  // plus the out_proj output's staging slabs: 8 waves x 32 rows x 80 bytes
  const int64_t lds = gate32_lds_bytes(a.Kp, o.ldq, 3, 8, a.out_dt == kBF16) + 8 * 32 * 80;
  if (dl.cus <= 0 || lds > dl.lds) return -1;
  G32Out op;
  op.w = out_proj.w;
  op.ldw = out_proj.ldw;
  op.c_w = out_proj.c_w;
  op.out = out;
  op.ldo = ldout;
  if (nks == 4)
    launch_gate32<8, 3, 4, 24>(a, o, lds, st, op);
  else if (nks == 8)
    launch_gate32<8, 3, 8, 24>(a, o, lds, st, op);
  else
    launch_gate32<8, 3, 12, 24>(a, o, lds, st, op);
  return check_launch("output gate + out_proj (32-row tiles)");
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
  if (const int rc = try_gate32(a, o, st); rc >= 0) return rc;
  const int64_t tiles = (a.N + 15) / 16;
  if (tiles <= 4) return run_rowq<4, 1>(a, o, st);
  if (tiles <= 8) return run_rowq<4, 2>(a, o, st);
  if (tiles <= 12) return run_rowq<4, 3>(a, o, st);
  if (tiles <= 16) return run_rowq<4, 4>(a, o, st);
  if (tiles <= 24) return run_rowq<8, 3>(a, o, st);
  if (tiles <= 32) return run_rowq<8, 4>(a, o, st);
  if (tiles <= 48) return run_rowq<8, 6>(a, o, st);
  return run_rowq<8, 8>(a, o, st);
}

}  // namespace tesm
