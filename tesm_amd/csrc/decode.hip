// TESM_SISO / TESMMIMO_Optimized one-token decode step and the decode caches written by a prefill.
//
// Reference semantics (tesm_ssm/modules/tesm.py, tesm_mimo.py):
//   decode step      _forward_incremental, tesm.py:1274-1400; MIMO per head, tesm_mimo.py:753-912
//   prefill caches   TESM_SISO.forward, tesm.py:1235-1253
//   cache layout     allocate_inference_cache, tesm.py:620-670; MIMO (B, W, H, .), tesm_mimo.py:689-731
//
// One workgroup per (batch row, head); SISO is the one-head case.  The MIMO step has no rank
// expansion (tesm_mimo.py:827-829): each head is a SISO step with its own decay-bias and window-bias
// rows, and the per-token quantization of tanh(E) and C spans all heads, so that step writes E's
// values and a row quantization follows.
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

constexpr int kDecMaxCPT = 8;  // channels per thread: at most 2048 channels per workgroup

// Raw bits of four consecutive ring values at p[i .. i+3] (16-byte aligned for f32, 8-byte for bf16):
// f32 four words, bf16 two words of two values each (ring_val reads them back).
template <int CDT>
__device__ __forceinline__ void ld4_bits(const void* p, int64_t i, uint32_t (&r)[4]) {
  if constexpr (CDT == kBF16) {
    const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p) + i);
    r[0] = w.x;
    r[1] = w.y;
    r[2] = 0;
    r[3] = 0;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const float*>(p) + i);
    r[0] = w.x;
    r[1] = w.y;
    r[2] = w.z;
    r[3] = w.w;
  }
}

// Value e (0..3) of four ring values read by ld4_bits (vec) or as four single elements (ld_bits).
template <int CDT>
__device__ __forceinline__ float ring_val(const uint32_t (&r)[4], int e, bool vec) {
  if constexpr (CDT == kBF16) {
    if (vec) return __uint_as_float(e & 1 ? r[e >> 1] & 0xffff0000u : r[e >> 1] << 16);
    return __uint_as_float(r[e] << 16);
  } else {
    return __uint_as_float(r[e]);
  }
}

// Workgroup (b, h, z) owns channels [z*chunk, z*chunk + chunk) of head h of batch row b.  Every
// workgroup of a head computes the same query, key, window scores and weights (the key ring is
// read once per chunk); the state update, ring write of the state, mix and outputs are per channel.
// The key goes into the ring from chunk 0 only.  Reads of the ring skip this step's slot, whose
// fresh key / state come from LDS, so the ring writes of other workgroups never race a read.
// Window keys are loaded four windows at a time; ring slots and offsets are formed in 32-bit
// arithmetic.  CPT: channels per thread.  With CPT = 1 (chunks of at most 256 channels) lane l of
// wave v holds channels 4l .. 4l+3 of the chunk at window positions v, v+4, .. (vector loads
// requested at the start, so they overlap the RoPE, state update and scores), and the four waves'
// partial mixes are added in a fixed order; with CPT = kDecMaxCPT (up to 2048 channels) each thread
// sums its channels' positions in order, four positions' loads at a time.  NI: rank elements per
// lane and half (ent_rank <= 128 * NI).
// FUSE: one head and one chunk (SISO): the int8 codes of tanh(E) and C are formed here; otherwise
// tanh(E) and C are written in dt to te_out / c_out (row b, columns h*D + c).
template <int DT, int CDT, bool FUSE, int CPT, int NI>
__global__ __launch_bounds__(256) void decode_ent_kernel(DecodeArgs a) {
  extern __shared__ __attribute__((aligned(16))) float lds_dec[];
  const int R = static_cast<int>(a.R), W = static_cast<int>(a.W), CW = static_cast<int>(a.chunk);
  const int D = static_cast<int>(a.D);
  const int half = R / 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t b = blockIdx.x, h = blockIdx.y, H = a.H;
  const int c0 = static_cast<int>(blockIdx.z) * CW;
  const int cn = min(CW, D - c0);  // channels of this workgroup (>= 1)
  float* qv = lds_dec;       // R   RoPE'd query (+ cross query)
  float* kv = qv + R;        // R   RoPE'd key of this step
  float* nv = kv + R;        // CW  new state of this chunk in the layer dtype
  float* wn = nv + CW;       // 64  window bias, then ternary / norm per padded window position
  float* red = wn + 64;      // 16  block reductions
  int* redi = reinterpret_cast<int*>(red + 8);
  float* mixp = red + 16;    // 4 x CW  per-wave partial mixes (CPT = 1)
  const int64_t bh = b * H + h;  // row of the (B, H, .) state, cross query and new state
  const int es = DT == kBF16 ? 2 : 4;
  const char* prow = static_cast<const char*>(a.proj) + b * a.ld_proj * es;
  const int64_t o_q = a.o_q + h * a.R, o_k = a.o_k + h * a.R;
  const int64_t o_sv = a.o_sv + h * a.D, o_decay = a.o_decay + h * a.D, o_write = a.o_write + h * a.D;
  const float* wbias = a.bias + h * a.W;
  // ring element (b, s, h, i): keys at kbase + s*kstep + i, states at vbase + s*vstep + i
  const int64_t kbase = (b * a.W * H + h) * a.R, kstep = H * a.R;
  const int64_t vbase = (b * a.W * H + h) * a.D + c0, vstep = H * a.D;
  int64_t pos = a.pos;
  int slot = static_cast<int>(a.slot), valid = static_cast<int>(a.valid);
  if (a.step_pos) {  // position kept on the device (graph replay): read it here
    const int64_t sp = a.step_pos[0] < 0 ? 0 : a.step_pos[0], si = a.step_pos[1] % W;
    pos = sp < a.rope_rows ? sp : a.rope_rows - 1;
    slot = static_cast<int>(si < 0 ? si + W : si);
    valid = static_cast<int>(sp + 1 < W ? sp + 1 : W);
  }
  const int wlo = W - valid;  // padded positions below wlo hold no entry
  const bool full = valid >= W;
  // ring slot read at padded window position w (w in [wlo, W)), in the reference's order; selects
  // rather than branches (the value for other w is not used)
  auto slot_of = [&](int w) -> int {
    const int s = full ? slot + w : w - wlo;
    return s >= W ? s - W : s;
  };

  // Ring slot the loads for window position w read: the position's slot, or for positions without a
  // ring entry (padding, past W) and for this step's slot (its key and state come from LDS) another
  // slot, so the loads need no branch and, with W > 1, never read the slot this step writes.
  const int alt = W > 1 ? (slot + 1 == W ? 0 : slot + 1) : slot;
  auto read_slot = [&](int w) -> int {
    const int s = slot_of(w);
    return ((w >= wlo) & (w < W) & (s != slot)) ? s : alt;
  };

  // 0. Every global read of steps 1-4 (the last batches of window keys and, with CPT > 1, of ring
  //    states aside) is issued here in straight-line code, indices clamped into range and values at
  //    unused positions discarded, and converted where used: the workgroup waits for memory about
  //    once instead of once per guarded load.
  // 0a. (CPT = 1) ring states of this thread's four channels at its window positions
  const int j4 = 4 * lane;
  const bool vec = a.vec4 != 0;  // chunk widths are multiples of 4 and ring rows aligned
  uint32_t xr[CPT == 1 ? 16 : 1][4];
  if constexpr (CPT == 1) {
    if (vec) {
      const int jc = min(j4, cn - 4);
#pragma unroll
      for (int u = 0; u < 16; ++u) {  // W <= 64
        const int w = wave + 4 * u;
        if (w >= W) break;  // uniform in the wave
        ld4_bits<CDT>(a.v_cache, vbase + static_cast<int64_t>(read_slot(w)) * vstep + jc, xr[u]);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int w = wave + 4 * u;
        if (w >= W) break;
        const int64_t vo = vbase + static_cast<int64_t>(read_slot(w)) * vstep;
#pragma unroll
        for (int r = 0; r < 4; ++r) xr[u][r] = ld_bits<CDT>(a.v_cache, vo + min(j4 + r, cn - 1));
      }
    }
  }
  // 0b. RoPE inputs of element tid of each rank half (half <= 256)
  const int ir = tid < half ? tid : half - 1;
  const float2 rcs = a.rope[pos * half + ir];
  const uint32_t bq1 = ld_bits<DT>(prow, o_q + ir), bq2 = ld_bits<DT>(prow, o_q + half + ir);
  const uint32_t bk1 = ld_bits<DT>(prow, o_k + ir), bk2 = ld_bits<DT>(prow, o_k + half + ir);
  const void* qadd = a.q_add ? a.q_add : a.proj;  // no cross query: a valid dummy address
  const int64_t qo = a.q_add ? bh * a.ld_qadd : 0;
  const uint32_t ba1 = ld_bits<DT>(qadd, qo + ir), ba2 = ld_bits<DT>(qadd, qo + half + ir);
  const float wbv = wbias[tid < W ? tid : W - 1];  // window bias of position tid, parked in wn below
  // 0c. gate inputs and float64 state of the thread's channels
  uint32_t bdc[CPT], bdb[CPT], bwr[CPT], bsv[CPT];
  double st64[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int j = tid + 256 * k, c = c0 + (j < cn ? j : cn - 1);
    bdc[k] = ld_bits<DT>(prow, o_decay + c);
    bdb[k] = ld_bits<DT>(a.decay_bias, h * a.D + c);
    bwr[k] = ld_bits<DT>(prow, o_write + c);
    bsv[k] = ld_bits<DT>(prow, o_sv + c);
    st64[k] = a.state[bh * a.D + c];
  }
  // 0d. window keys of the wave's first four window positions (later batches in step 3)
  uint32_t kb[4][2 * NI];
  auto load_keys = [&](int j0) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int64_t ko = kbase + static_cast<int64_t>(read_slot(wave + 4 * (j0 + jj))) * kstep;
#pragma unroll
      for (int t = 0; t < NI; ++t) {
        const int i = min(lane + 64 * t, half - 1);
        kb[jj][2 * t] = ld_bits<CDT>(a.k_cache, ko + i);
        kb[jj][2 * t + 1] = ld_bits<CDT>(a.k_cache, ko + half + i);
      }
    }
  };
  load_keys(0);

  // 1. RoPE at position pos (tesm.py:1311-1313), cross query (1302-1305), key into the ring
  if (tid < W) wn[tid] = wbv;  // read back (and replaced by the ternary) by the lane scoring position tid
  if (tid < half) {
    float q1, q2, k1, k2;
    rope_pair<DT>(from_bits<DT>(bq1), from_bits<DT>(bq2), rcs, q1, q2);
    rope_pair<DT>(from_bits<DT>(bk1), from_bits<DT>(bk2), rcs, k1, k2);
    if (a.q_add) {
      q1 = rnd<DT>(q1 + from_bits<DT>(ba1));
      q2 = rnd<DT>(q2 + from_bits<DT>(ba2));
    }
    qv[tid] = q1;
    qv[half + tid] = q2;
    kv[tid] = k1;
    kv[half + tid] = k2;
    if (blockIdx.z == 0) {
      const int64_t ko = kbase + slot * kstep;
      st<CDT>(a.k_cache, ko + tid, k1);
      st<CDT>(a.k_cache, ko + half + tid, k2);
    }
  }
  // 2. gates and the float64 state update (tesm.py:1315-1322): new = decay * h + write * tanh(sv)
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int j = tid + 256 * k;
    if (j >= cn) continue;
    const int c = c0 + j;
    const float d = rnd<DT>(sigmoidf_(rnd<DT>(from_bits<DT>(bdc[k]) + from_bits<DT>(bdb[k]))));
    const float wr = rnd<DT>(sigmoidf_(from_bits<DT>(bwr[k])));
    const float sv = rnd<DT>(tanhf_(from_bits<DT>(bsv[k])));
    const double n64 = static_cast<double>(d) * st64[k] + static_cast<double>(wr) * static_cast<double>(sv);
    a.state_out[bh * a.D + c] = n64;
    const float nf = rnd<DT>(static_cast<float>(n64));  // torch: float64 -> float -> dtype
    nv[j] = nf;
    st<CDT>(a.v_cache, vbase + slot * vstep + j, nf);
    if (a.new_state) st<DT>(a.new_state, bh * a.D + c, nf);
  }
  __syncthreads();

  // 3. window scores (tesm.py:1338-1357): wave v scores windows v, v+4, ..; its lanes split the rank.
  //    A batch's four dot products are formed and reduced together (the next batch's keys requested
  //    first), then lane jj turns window jj's sum into its ternary.  The step's own query and key
  //    values come from LDS once; the fresh window picks the key by a select, lanes past the rank add
  //    zero.
  const float sq = static_cast<float>(sqrt(static_cast<double>(a.R)));
  float q1v[NI], q2v[NI], k1v[NI], k2v[NI];
#pragma unroll
  for (int t = 0; t < NI; ++t) {
    const int i = min(lane + 64 * t, half - 1);
    q1v[t] = qv[i];
    q2v[t] = qv[half + i];
    k1v[t] = kv[i];
    k2v[t] = kv[half + i];
  }
  for (int j0 = 0; j0 < 16; j0 += 4) {  // W <= 64: at most 16 windows per wave
    if (wave + 4 * j0 >= W) break;       // uniform in the wave
    float dot[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const bool fresh = slot_of(wave + 4 * (j0 + jj)) == slot;  // (value unused off the window)
      float d = 0.0f;
#pragma unroll
      for (int t = 0; t < NI; ++t) {
        const bool in = lane + 64 * t < half;
        const float k1 = fresh ? k1v[t] : rnd<DT>(from_bits<CDT>(kb[jj][2 * t]));
        const float k2 = fresh ? k2v[t] : rnd<DT>(from_bits<CDT>(kb[jj][2 * t + 1]));
        d += in ? q1v[t] * k1 : 0.0f;
        d += in ? q2v[t] * k2 : 0.0f;
      }
      dot[jj] = d;
    }
    if (j0 + 4 < 16 && wave + 4 * (j0 + 4) < W) load_keys(j0 + 4);  // uniform in the wave
    wave_sum_fn<4>(dot);
    const int w = wave + 4 * (j0 + (lane & 3));
    if (lane < 4 && w < W) {
      const float dsum = lane == 0 ? dot[0] : (lane == 1 ? dot[1] : (lane == 2 ? dot[2] : dot[3]));
      if (w < wlo) {
        wn[w] = 0.0f;
      } else {
        float sc = rnd<DT>(rnd<DT>(dsum) / sq);
        sc = rnd<DT>(sc + wn[w]);  // wn[w] holds the window bias until here
        wn[w] = sc > a.thr ? 1.0f : (sc < -a.thr ? -1.0f : 0.0f);  // strict ternary (1359-1368)
      }
    }
  }
  __syncthreads();
  if (wave == 0) {  // count normalisation (1370-1372)
    const float tern = lane < W ? wn[lane] : 0.0f;
    float cnt[1] = {fabsf(tern)};
    wave_sum_fn<1>(cnt);  // a count: exact in any order
    const float n = fmaxf(cnt[0], 1.0f);
    if (lane < W) wn[lane] = rnd<DT>(tern / n);
    if (a.tern && blockIdx.z == 0 && lane < W) a.tern[bh * a.W + lane] = static_cast<int8_t>(tern);
  }
  __syncthreads();

  // 4. mix, entangled state, tanh(E) and C = E - S (tesm.py:1373-1390)
  float acc[CPT];
#pragma unroll
  for (int k = 0; k < CPT; ++k) acc[k] = 0.0f;
  if constexpr (CPT == 1) {
    float pm[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    float nvr[4];  // this step's states of the lane's channels (the fresh window), picked by a select
#pragma unroll
    for (int r = 0; r < 4; ++r) nvr[r] = nv[min(j4 + r, cn - 1)];  // channels past cn are not stored
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int w = wave + 4 * u;
      if (w >= W) break;  // uniform in the wave
      if (w < wlo) continue;
      const bool fresh = slot_of(w) == slot;
      const float wv = wn[w];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = fresh ? nvr[r] : rnd<DT>(ring_val<CDT>(xr[u], r, vec));
        pm[r] += wv * x;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (j4 + r < cn) mixp[wave * CW + j4 + r] = pm[r];
    __syncthreads();
    if (tid < cn) acc[0] = ((mixp[tid] + mixp[CW + tid]) + mixp[2 * CW + tid]) + mixp[3 * CW + tid];
  } else {
    constexpr int kWB = 4;
    float nvk[CPT];  // this step's states of the thread's channels (the fresh window)
#pragma unroll
    for (int k = 0; k < CPT; ++k) nvk[k] = nv[min(tid + 256 * k, cn - 1)];  // channels past cn are not stored
    for (int w0 = wlo; w0 < W; w0 += kWB) {
      uint32_t xb[kWB][CPT];  // a batch's loads in straight-line code, all in flight together
#pragma unroll
      for (int u = 0; u < kWB; ++u) {
        const int64_t vo = vbase + static_cast<int64_t>(read_slot(w0 + u)) * vstep;
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          const int j = tid + 256 * k;
          xb[u][k] = ld_bits<CDT>(a.v_cache, vo + (j < cn ? j : cn - 1));
        }
      }
#pragma unroll
      for (int u = 0; u < kWB; ++u) {
        const int w = w0 + u;
        if (w >= W) break;
        const bool fresh = slot_of(w) == slot;
        const float wv = wn[w];
#pragma unroll
        for (int k = 0; k < CPT; ++k) {
          const float x = fresh ? nvk[k] : rnd<DT>(from_bits<CDT>(xb[u][k]));
          acc[k] += wv * x;
        }
      }
    }
  }
  float tv[CPT], cv[CPT];
  float mx_t = 0.0f, mx_c = 0.0f;
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int j = tid + 256 * k;
    tv[k] = 0.0f;
    cv[k] = 0.0f;
    if (j >= cn) continue;
    const float avg = rnd<DT>(acc[k]);
    const float sv = nv[j];
    const float ev = rnd<DT>(sv + rnd<DT>(a.ent_scale * rnd<DT>(avg - sv)));
    cv[k] = rnd<DT>(ev - sv);
    tv[k] = rnd<DT>(tanhf_(ev));
    mx_t = fmaxf(mx_t, fabsf(tv[k]));
    mx_c = fmaxf(mx_c, fabsf(cv[k]));
  }
  if constexpr (!FUSE) {  // MIMO: the row quantization spans the heads
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int j = tid + 256 * k;
      if (j >= cn) continue;
      st<DT>(a.te_out, b * a.ld_out + h * a.D + c0 + j, tv[k]);
      st<DT>(a.c_out, b * a.ld_out + h * a.D + c0 + j, cv[k]);
    }
    return;
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
  for (int k = 0; k < CPT; ++k) {
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

__global__ void decode_advance_kernel(int64_t* __restrict__ sp, int64_t W) {
  if (threadIdx.x == 0) {
    sp[0] += 1;
    sp[1] = (sp[1] + 1) % W;
  }
}

}  // namespace

int launch_decode_advance(int64_t* step_pos, int64_t W, hipStream_t st) {
  TESM_REQUIRE(step_pos && W >= 1, kErrInvalidArg, "decode advance: bad arguments");
  decode_advance_kernel<<<1, 64, 0, TESM_LOGGED(st, decode_advance_kernel)>>>(step_pos, W);
  return check_launch("decode advance");
}

int64_t decode_lds_bytes(int64_t R, int64_t CW) { return (2 * R + 5 * CW + 64 + 16) * static_cast<int64_t>(sizeof(float)); }

int launch_decode_ent(const DecodeArgs& a, hipStream_t st) {
  TESM_REQUIRE(a.dt == kF32 || a.dt == kBF16, kErrInvalidArg, "decode: dtype must be 0 or 1");
  TESM_REQUIRE(a.cdt == kF32 || a.cdt == kBF16, kErrInvalidArg, "decode: cache dtype must be 0 or 1");
  TESM_REQUIRE(a.B >= 1 && a.R >= 2 && a.R % 2 == 0 && a.D >= 1, kErrInvalidArg, "decode: bad sizes");
  TESM_REQUIRE(a.R <= 512, kErrUnsupported, "decode: ent_rank must be <= 512");
  TESM_REQUIRE(a.W >= 1 && a.W <= 64, kErrUnsupported, "decode: window must be in [1, 64]");
  TESM_REQUIRE(a.valid >= 1 && a.valid <= a.W && a.slot >= 0 && a.slot < a.W, kErrInvalidArg,
               "decode: bad ring position");
  TESM_REQUIRE(a.proj && a.rope && a.decay_bias && a.bias && a.state && a.state_out && a.k_cache && a.v_cache,
               kErrInvalidArg, "decode: null pointer");
  TESM_REQUIRE(a.H >= 1 && a.H <= 65535, kErrInvalidArg, "decode: bad head count");
  const bool fuse = a.q_te != nullptr;
  if (fuse) {
    TESM_REQUIRE(a.H == 1, kErrInvalidArg, "decode: fused codes need one head");
    TESM_REQUIRE(a.D <= 256 * kDecMaxCPT, kErrUnsupported, "decode: d_state must be <= 2048");
    TESM_REQUIRE(a.q_c && a.s_te && a.s_c && a.rs_te && a.rs_c, kErrInvalidArg, "decode: null pointer");
    TESM_REQUIRE(a.ldq >= a.D, kErrInvalidArg, "decode: ldq < d_state");
  } else {
    TESM_REQUIRE(a.te_out && a.c_out && a.ld_out >= a.H * a.D, kErrInvalidArg,
                 "decode: need te_out / c_out with ld_out >= n_heads * d_state");
  }
  // channel chunks: one per workgroup for the fused (one-head) step; otherwise enough chunks of at
  // least 128 channels for about 1024 workgroups
  int64_t nz = 1;
  if (!fuse) {
    const int64_t want = (1024 + a.B * a.H - 1) / (a.B * a.H);
    nz = std::max<int64_t>(1, std::min<int64_t>(want, (a.D + 127) / 128));
  }
  int64_t cw = (a.D + nz - 1) / nz;
  nz = (a.D + cw - 1) / cw;  // every chunk non-empty
  TESM_REQUIRE(cw <= 256 * kDecMaxCPT && nz <= 65535, kErrUnsupported, "decode: d_state too large");
  DecodeArgs k = a;
  k.chunk = cw;
  k.vec4 = a.D % 4 == 0 && cw % 4 == 0 && aligned(a.v_cache, a.cdt == kBF16 ? 8 : 16);
  const size_t lds = static_cast<size_t>(decode_lds_bytes(a.R, cw));
  const dim3 grid(static_cast<unsigned>(a.B), static_cast<unsigned>(a.H), static_cast<unsigned>(nz));
  const bool cpt1 = cw <= 256;
  const int ni = a.R <= 128 ? 1 : (a.R <= 256 ? 2 : 4);
#define TESM_DEC_LAUNCH3(DT_, CDT_, FUSE_, CPT_)                                        \
  do {                                                                                 \
    if (ni == 1)                                                                       \
      decode_ent_kernel<DT_, CDT_, FUSE_, CPT_, 1><<<grid, 256, lds, TESM_LOGGED(st, decode_ent_kernel<DT_, CDT_, FUSE_, CPT_, 1>)>>>(k);         \
    else if (ni == 2)                                                                  \
      decode_ent_kernel<DT_, CDT_, FUSE_, CPT_, 2><<<grid, 256, lds, TESM_LOGGED(st, decode_ent_kernel<DT_, CDT_, FUSE_, CPT_, 2>)>>>(k);         \
    else                                                                               \
      decode_ent_kernel<DT_, CDT_, FUSE_, CPT_, 4><<<grid, 256, lds, TESM_LOGGED(st, decode_ent_kernel<DT_, CDT_, FUSE_, CPT_, 4>)>>>(k);         \
  } while (0)
#define TESM_DEC_LAUNCH2(DT_, CDT_, FUSE_)                                             \
  do {                                                                                 \
    if (cpt1)                                                                          \
      TESM_DEC_LAUNCH3(DT_, CDT_, FUSE_, 1);                                           \
    else                                                                               \
      TESM_DEC_LAUNCH3(DT_, CDT_, FUSE_, kDecMaxCPT);                                  \
  } while (0)
#define TESM_DEC_LAUNCH(DT_, CDT_)                                                     \
  do {                                                                                 \
    if (fuse)                                                                          \
      TESM_DEC_LAUNCH2(DT_, CDT_, true);                                               \
    else                                                                               \
      TESM_DEC_LAUNCH2(DT_, CDT_, false);                                              \
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
#undef TESM_DEC_LAUNCH2
#undef TESM_DEC_LAUNCH3
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
        cache_fill_kernel<kBF16, kBF16, kF32><<<grid, 256, 0, TESM_LOGGED(st, cache_fill_kernel<kBF16, kBF16, kF32>)>>>(a);
      else
        cache_fill_kernel<kBF16, kF32, kF32><<<grid, 256, 0, TESM_LOGGED(st, cache_fill_kernel<kBF16, kF32, kF32>)>>>(a);
    } else {
      if (a.cdt == kBF16)
        cache_fill_kernel<kBF16, kBF16, kBF16><<<grid, 256, 0, TESM_LOGGED(st, cache_fill_kernel<kBF16, kBF16, kBF16>)>>>(a);
      else
        cache_fill_kernel<kBF16, kF32, kBF16><<<grid, 256, 0, TESM_LOGGED(st, cache_fill_kernel<kBF16, kF32, kBF16>)>>>(a);
    }
  } else {
    if (a.cdt == kBF16)
      cache_fill_kernel<kF32, kBF16, kF32><<<grid, 256, 0, TESM_LOGGED(st, cache_fill_kernel<kF32, kBF16, kF32>)>>>(a);
    else
      cache_fill_kernel<kF32, kF32, kF32><<<grid, 256, 0, TESM_LOGGED(st, cache_fill_kernel<kF32, kF32, kF32>)>>>(a);
  }
  return check_launch("cache fill");
}

}  // namespace tesm
