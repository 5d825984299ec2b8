// TESM_SISO one-token decode step and the decode caches written by a prefill.
//
// Reference semantics (tesm_ssm/modules/tesm.py):
//   decode step      _forward_incremental, tesm.py:1274-1400
//   prefill caches   TESM_SISO.forward, tesm.py:1235-1253
//   cache layout     allocate_inference_cache, tesm.py:620-670
//
// The ring buffers hold W keys (post-RoPE) and W states per batch row.  A step writes the new key and
// state into slot `slot` and then reads the window in the reference's order: with a full ring
// (valid == W) slots slot, slot+1, ... (mod W) -- the newest entry first, meeting bias[0]; with a
// partial ring slots 0 .. valid-1.  Entry e of the window sits at padded position w = W - valid + e
// and meets bias[w].  Mixed-dtype reads follow the reference with its dtype amendment: cache entries
// are cast to the layer dtype (lossless, every entry is a layer-dtype value).
#include "decode.h"

namespace tesm {

namespace {

constexpr int kDecMaxCPT = 8;  // channels per thread: d_state <= 2048

// STG: the window's ring rows are copied to LDS at the start (keys at pitch R + 1 so the per-window
// dot products of one wave hit distinct banks), so their latency overlaps the RoPE and the state
// update instead of following them.
template <int DT, int CDT, bool STG>
__global__ __launch_bounds__(256) void decode_ent_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_dec[];
  const int R = static_cast<int>(a.R), D = static_cast<int>(a.D), W = static_cast<int>(a.W);
  const int half = R / 2;
  float* qv = lds_dec;       // R   RoPE'd query (+ cross query)
  float* kv = qv + R;        // R   RoPE'd key of this step
  float* nv = kv + R;        // D   new state in the layer dtype
  float* wn = nv + D;        // 64  ternary / norm per padded window position
  float* red = wn + 64;      // 16  block reductions
  int* redi = reinterpret_cast<int*>(red + 8);
  float* kw = red + 16;      // STG: W x (R + 1) ring keys in the layer dtype
  float* vw = kw + (STG ? W * (R + 1) : 0);  // STG: W x D ring states in the layer dtype
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t b = blockIdx.x;
  const int es = DT == kBF16 ? 2 : 4;
  const char* prow = static_cast<const char*>(a.proj) + b * a.ld_proj * es;
  const int64_t slot = a.slot;
  if constexpr (STG) {  // this step's slot is read too but never used: its fresh key / state come from kv / nv
    for (int i = tid; i < W * R; i += 256) {
      const int s = i / R, r = i - s * R;
      kw[s * (R + 1) + r] = rnd<DT>(ld<CDT>(a.k_cache, (b * a.W + s) * a.R + r));
    }
    for (int i = tid; i < W * D; i += 256) vw[i] = rnd<DT>(ld<CDT>(a.v_cache, b * a.W * a.D + i));
  }

  // 1. RoPE at position pos (tesm.py:1311-1313), cross query (1302-1305), key into the ring
  for (int i = tid; i < half; i += 256) {
    const float2 cs = a.rope[a.pos * half + i];
    float q1, q2, k1, k2;
    rope_pair<DT>(ld<DT>(prow, a.o_q + i), ld<DT>(prow, a.o_q + half + i), cs, q1, q2);
    rope_pair<DT>(ld<DT>(prow, a.o_k + i), ld<DT>(prow, a.o_k + half + i), cs, k1, k2);
    if (a.q_add) {
      q1 = rnd<DT>(q1 + ld<DT>(a.q_add, b * a.ld_qadd + i));
      q2 = rnd<DT>(q2 + ld<DT>(a.q_add, b * a.ld_qadd + half + i));
    }
    qv[i] = q1;
    qv[half + i] = q2;
    kv[i] = k1;
    kv[half + i] = k2;
    const int64_t ko = (b * a.W + slot) * a.R;
    st<CDT>(a.k_cache, ko + i, k1);
    st<CDT>(a.k_cache, ko + half + i, k2);
  }
  // 2. gates and the float64 state update (tesm.py:1315-1322): new = decay * h + write * tanh(sv)
  for (int c = tid; c < D; c += 256) {
    const float d = rnd<DT>(sigmoidf_(rnd<DT>(ld<DT>(prow, a.o_decay + c) + ld<DT>(a.decay_bias, c))));
    const float wr = rnd<DT>(sigmoidf_(ld<DT>(prow, a.o_write + c)));
    const float sv = rnd<DT>(tanhf_(ld<DT>(prow, a.o_sv + c)));
    const double n64 = static_cast<double>(d) * a.state[b * a.D + c] + static_cast<double>(wr) * static_cast<double>(sv);
    a.state_out[b * a.D + c] = n64;
    const float nf = rnd<DT>(static_cast<float>(n64));  // torch: float64 -> float -> dtype
    nv[c] = nf;
    st<CDT>(a.v_cache, (b * a.W + slot) * a.D + c, nf);
    if (a.new_state) st<DT>(a.new_state, b * a.D + c, nf);
  }
  __syncthreads();

  // 3. window scores, strict ternary, count normalisation (tesm.py:1338-1372); one wave
  const int64_t valid = a.valid;
  if (wave == 0) {
    const int w = lane;
    float tern = 0.0f;
    if (w < W && w >= W - valid) {
      const int64_t e = w - (W - valid);
      const int64_t s = a.full ? (slot + w) % a.W : e;
      float dot = 0.0f;
      for (int i = 0; i < half; ++i) {
        float k1, k2;
        if (s == slot) {
          k1 = kv[i];
          k2 = kv[half + i];
        } else if constexpr (STG) {
          k1 = kw[s * (R + 1) + i];
          k2 = kw[s * (R + 1) + half + i];
        } else {
          const int64_t ko = (b * a.W + s) * a.R;
          k1 = rnd<DT>(ld<CDT>(a.k_cache, ko + i));
          k2 = rnd<DT>(ld<CDT>(a.k_cache, ko + half + i));
        }
        dot += qv[i] * k1;
        dot += qv[half + i] * k2;
      }
      const float sq = static_cast<float>(sqrt(static_cast<double>(a.R)));
      float sc = rnd<DT>(rnd<DT>(dot) / sq);
      sc = rnd<DT>(sc + a.bias[w]);
      tern = sc > a.thr ? 1.0f : (sc < -a.thr ? -1.0f : 0.0f);
    }
    const float n = fmaxf(wave_sum_f<64>(fabsf(tern)), 1.0f);
    if (w < W) wn[w] = rnd<DT>(tern / n);
  }
  __syncthreads();

  // 4. mix, entangled state, tanh(E) and C = E - S (tesm.py:1373-1390)
  float tv[kDecMaxCPT], cv[kDecMaxCPT];
  float mx_t = 0.0f, mx_c = 0.0f;
#pragma unroll
  for (int k = 0; k < kDecMaxCPT; ++k) {
    const int c = tid + 256 * k;
    tv[k] = 0.0f;
    cv[k] = 0.0f;
    if (c >= D) continue;
    float acc = 0.0f;
    for (int w = static_cast<int>(W - valid); w < W; ++w) {
      const int64_t e = w - (W - valid);
      const int64_t s = a.full ? (slot + w) % a.W : e;
      float x;
      if (s == slot)
        x = nv[c];
      else if constexpr (STG)
        x = vw[s * D + c];
      else
        x = rnd<DT>(ld<CDT>(a.v_cache, (b * a.W + s) * a.D + c));
      acc += wn[w] * x;
    }
    const float avg = rnd<DT>(acc);
    const float sv = nv[c];
    const float ev = rnd<DT>(sv + rnd<DT>(a.ent_scale * rnd<DT>(avg - sv)));
    cv[k] = rnd<DT>(ev - sv);
    tv[k] = rnd<DT>(tanhf_(ev));
    mx_t = fmaxf(mx_t, fabsf(tv[k]));
    mx_c = fmaxf(mx_c, fabsf(cv[k]));
  }
  // 5. per-token int8 codes of tanh(E) and C for state_proj / ent_proj (tesm.py:206-209), layout 1
  mx_t = wave_max<64>(mx_t);
  mx_c = wave_max<64>(mx_c);
  if (lane == 0) {
    red[wave] = mx_t;
    red[4 + wave] = mx_c;
  }
  __syncthreads();
  mx_t = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  mx_c = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
  const float sc_t = act_scale<DT>(mx_t, a.eps);
  const float sc_c = act_scale<DT>(mx_c, a.eps);
  int sum_t = 0, sum_c = 0;
  int8_t* qt = a.q_te + b * a.ldq;
  int8_t* qc = a.q_c + b * a.ldq;
#pragma unroll
  for (int k = 0; k < kDecMaxCPT; ++k) {
    const int c = tid + 256 * k;
    if (c >= D) continue;
    const int c1 = act_code<DT>(tv[k], sc_t), c2 = act_code<DT>(cv[k], sc_c);
    sum_t += c1;
    sum_c += c2;
    const int pos = (c & ~15) + layout1_pos(c & 15);
    qt[pos] = static_cast<int8_t>(c1);
    qc[pos] = static_cast<int8_t>(c2);
  }
  for (int64_t c = D + tid; c < a.ldq; c += 256) {  // padding channels: code 0 at their layout-1 byte
    const int64_t pos = (c & ~static_cast<int64_t>(15)) + layout1_pos(static_cast<int>(c & 15));
    qt[pos] = 0;
    qc[pos] = 0;
  }
  sum_t = wave_sum_i<64>(sum_t);
  sum_c = wave_sum_i<64>(sum_c);
  if (lane == 0) {
    redi[wave] = sum_t;
    redi[4 + wave] = sum_c;
  }
  __syncthreads();
  if (tid == 0) {
    a.s_te[b] = sc_t;
    a.rs_te[b] = (redi[0] + redi[1]) + (redi[2] + redi[3]);
    a.s_c[b] = sc_c;
    a.rs_c[b] = (redi[4] + redi[5]) + (redi[6] + redi[7]);
  }
}

// Prefill cache fill (tesm.py:1244-1251; MIMO tesm_mimo.py:1022-1037): rows t in [L - n, L),
// n = min(L, W), go to slot t - L + W, keys RoPE'd at position t (per head), states as computed
// (MIMO: the rank-0 states, S * vscale).
template <int DT, int CDT, int SDT>
__global__ __launch_bounds__(256) void cache_fill_kernel(CacheFillArgs a) {
  const int64_t n = a.L < a.W ? a.L : a.W;
  const int64_t r = blockIdx.x, b = blockIdx.y;  // r < n
  const int64_t t = a.L - n + r, slot = t - a.L + a.W;
  const int half = static_cast<int>(a.R / 2);
  const int64_t row = b * a.L + t;
  const int64_t HR = a.H * a.R, HD = a.H * a.D;
  for (int i = threadIdx.x; i < a.H * half; i += 256) {
    const int h = i / half, p = i - h * half;
    const int64_t ki = row * a.ld_k + h * a.R + p;
    float k1, k2;
    rope_pair<DT>(ld<DT>(a.k, ki), ld<DT>(a.k, ki + half), a.rope[t * half + p], k1, k2);
    const int64_t ko = (b * a.W + slot) * HR + h * a.R + p;
    st<CDT>(a.k_cache, ko, k1);
    st<CDT>(a.k_cache, ko + half, k2);
  }
  for (int64_t c = threadIdx.x; c < HD; c += 256) {
    float v = ld<SDT>(a.states, row * a.ld_states + c);
    if (a.vscale) v *= a.vscale[c];
    st<CDT>(a.v_cache, (b * a.W + slot) * HD + c, v);
  }
}

}  // namespace

int64_t decode_lds_bytes(int64_t R, int64_t D) { return (2 * R + D + 64 + 16) * static_cast<int64_t>(sizeof(float)); }

namespace {
constexpr int64_t kDecStageMax = 64 * 1024;  // LDS bytes up to which the ring rows are staged
int64_t decode_stage_bytes(int64_t R, int64_t D, int64_t W) {
  return decode_lds_bytes(R, D) + (W * (R + 1) + W * D) * static_cast<int64_t>(sizeof(float));
}
}  // namespace

int launch_decode_ent(const DecodeArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "decode: dtype must be 0 or 1");
  TESM_REQUIRE(a.cdt == kF32 || a.cdt == kBF16, kErrInvalidArg, "decode: cache dtype must be 0 or 1");
  TESM_REQUIRE(a.B >= 1 && a.R >= 2 && a.R % 2 == 0 && a.D >= 1, kErrInvalidArg, "decode: bad sizes");
  TESM_REQUIRE(a.D <= 256 * kDecMaxCPT, kErrUnsupported, "decode: d_state must be <= 2048");
  TESM_REQUIRE(a.W >= 1 && a.W <= 64, kErrUnsupported, "decode: window must be in [1, 64]");
  TESM_REQUIRE(a.valid >= 1 && a.valid <= a.W && a.slot >= 0 && a.slot < a.W, kErrInvalidArg,
               "decode: bad ring position");
  TESM_REQUIRE(a.proj && a.rope && a.decay_bias && a.bias && a.state && a.state_out && a.k_cache && a.v_cache && a.q_te &&
                   a.q_c && a.s_te && a.s_c && a.rs_te && a.rs_c,
               kErrInvalidArg, "decode: null pointer");
  TESM_REQUIRE(a.ldq >= a.D, kErrInvalidArg, "decode: ldq < d_state");
  const bool stg = decode_stage_bytes(a.R, a.D, a.W) <= kDecStageMax;
  const size_t lds = static_cast<size_t>(stg ? decode_stage_bytes(a.R, a.D, a.W) : decode_lds_bytes(a.R, a.D));
  const dim3 grid(static_cast<unsigned>(a.B));
#define TESM_DEC_LAUNCH(DT_, CDT_)                                                     \
  do {                                                                                 \
    if (stg)                                                                           \
      decode_ent_kernel<DT_, CDT_, true><<<grid, 256, lds, st>>>(a);                   \
    else                                                                               \
      decode_ent_kernel<DT_, CDT_, false><<<grid, 256, lds, st>>>(a);                  \
  } while (0)
  if (a.dt == kBF16) {
    if (a.cdt == kBF16)
      TESM_DEC_LAUNCH(kBF16, kBF16);
    else
      TESM_DEC_LAUNCH(kBF16, kF32);
  } else {
    if (a.cdt == kBF16)
      TESM_DEC_LAUNCH(kF32, kBF16);
    else
      TESM_DEC_LAUNCH(kF32, kF32);
  }
#undef TESM_DEC_LAUNCH
  return check_launch("decode step");
}

int launch_cache_fill(const CacheFillArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "cache fill: dtype must be 0 or 1");
  TESM_REQUIRE(a.cdt == kF32 || a.cdt == kBF16, kErrInvalidArg, "cache fill: cache dtype must be 0 or 1");
  TESM_REQUIRE(a.k && a.states && a.rope && a.k_cache && a.v_cache, kErrInvalidArg, "cache fill: null pointer");
  TESM_REQUIRE(a.W >= 1 && a.R % 2 == 0 && a.H >= 1, kErrInvalidArg, "cache fill: bad sizes");
  if (a.B == 0 || a.L == 0) return kOk;
  const int64_t n = a.L < a.W ? a.L : a.W;
  const dim3 grid(static_cast<unsigned>(n), static_cast<unsigned>(a.B));
  const int sdt = a.sdt < 0 ? a.dt : a.sdt;
  TESM_REQUIRE(sdt == a.dt || sdt == kF32, kErrUnsupported, "cache fill: states must be in dt or f32");
  if (a.dt == kBF16) {
    if (sdt == kF32) {
      if (a.cdt == kBF16)
        cache_fill_kernel<kBF16, kBF16, kF32><<<grid, 256, 0, st>>>(a);
      else
        cache_fill_kernel<kBF16, kF32, kF32><<<grid, 256, 0, st>>>(a);
    } else {
      if (a.cdt == kBF16)
        cache_fill_kernel<kBF16, kBF16, kBF16><<<grid, 256, 0, st>>>(a);
      else
        cache_fill_kernel<kBF16, kF32, kBF16><<<grid, 256, 0, st>>>(a);
    }
  } else {
    if (a.cdt == kBF16)
      cache_fill_kernel<kF32, kBF16, kF32><<<grid, 256, 0, st>>>(a);
    else
      cache_fill_kernel<kF32, kF32, kF32><<<grid, 256, 0, st>>>(a);
  }
  return check_launch("cache fill");
}

}  // namespace tesm
