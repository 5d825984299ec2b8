// extern "C" entry points of libtesm_hip.so (declared in include/tesm_hip.h) and the fused
// layer drivers.  The drivers only queue kernels on the caller's stream; every buffer comes
// from the caller (outputs) or from one caller-provided workspace carved up here.
#include <cxxabi.h>

#include <cctype>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>

#include "decode.h"
#include "entangle.h"
#include "global.h"
#include "mimo.h"
#include "norm.h"
#include "scan.h"
#include "tesm_hip_internal.h"
#include "../../include/tesm_hip.h"

namespace tesm {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int g_launch_log_on = 0;

namespace {
std::mutex g_log_mu;
std::string g_log;
}  // namespace

// "void tesm::(anonymous namespace)::name_kernel<1, 2, true>(tesm::Args)" -> "name_kernel<1,2,true>"
std::string short_kernel_name(const std::string& full) {
  const size_t pos = full.find("_kernel");
  if (pos == std::string::npos) return full;
  size_t b = pos;
  while (b > 0 && (std::isalnum(static_cast<unsigned char>(full[b - 1])) || full[b - 1] == '_')) --b;
  size_t e = pos + 7;
  if (e < full.size() && full[e] == '<') {
    int depth = 0;
    for (; e < full.size(); ++e) {
      if (full[e] == '<') ++depth;
      if (full[e] == '>' && --depth == 0) {
        ++e;
        break;
      }
    }
  }
  std::string out;
  for (size_t i = b; i < e && i < full.size(); ++i)
    if (full[i] != ' ') out += full[i];
  return out;
}

void log_kernel(const void* host_stub) {
  const char* mangled = hipKernelNameRefByPtr(host_stub, nullptr);
  std::string name = mangled ? mangled : "unknown_kernel";
  int status = 0;
  char* dem = abi::__cxa_demangle(name.c_str(), nullptr, nullptr, &status);
  if (status == 0 && dem) name = dem;
  std::free(dem);
  name = short_kernel_name(name);
  std::lock_guard<std::mutex> g(g_log_mu);
  g_log += name;
  g_log += '\n';
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(kErrLaunch, std::string(what) + ": launch failed: " + hipGetErrorString(e));
  return kOk;
}

namespace {

// Bump allocator over the caller's workspace (256-byte aligned pieces).
struct Carve {
  char* base;
  int64_t off = 0;
  explicit Carve(void* p) : base(static_cast<char*>(p)) {}
  template <class T>
  T* take(int64_t bytes) {
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off += round_up(std::max<int64_t>(bytes, 1), 256);
    return p;
  }
};

struct CodeBuf {
  int8_t* q;
  float* s;
  int32_t* rs;
  int64_t ldq;
};

CodeBuf take_codes(Carve& c, int64_t M, int64_t K) {
  CodeBuf b;
  b.ldq = kpad(K);
  b.q = c.take<int8_t>(M * b.ldq);
  b.s = c.take<float>(M * 4);
  b.rs = c.take<int32_t>(M * 4);
  return b;
}

// Per-token codes of tanh(E) and C (both (M, K), row pitch K) in one launch where their code buffers
// share a pitch, else one launch each.
static int quant_te_c(const void* te, const void* cc, int dt, int64_t M, int64_t K, float eps, const CodeBuf& xe,
                      const CodeBuf& xc, hipStream_t st) {
  if (xe.ldq == xc.ldq)
    return launch_quant_act2(te, cc, dt, M, K, K, eps, xe.q, xc.q, xe.ldq, xe.s, xc.s, xe.rs, xc.rs, st);
  if (int rc = launch_quant_act(te, dt, M, K, K, eps, 1, xe.q, xe.ldq, xe.s, xe.rs, st)) return rc;
  return launch_quant_act(cc, dt, M, K, K, eps, 1, xc.q, xc.ldq, xc.s, xc.rs, st);
}

LinearOperand operand(const CodeBuf& x, const tesm_hip_linear& w) {
  LinearOperand o;
  o.q = x.q;
  o.ldq = x.ldq;
  o.s_x = x.s;
  o.rowsum = x.rs;
  o.w = w.packed;
  o.ldw = w.ldw;
  o.c_w = w.c_w;
  o.c_w_per_row = w.c_w_per_row;
  return o;
}

int esize(int dt) { return dt == kBF16 ? 2 : 4; }

// Every pointer an entry point hands to a kernel must be memory the GPU can address: a device or
// managed allocation, or pinned host memory.  A pageable host pointer would make the kernel fault,
// so it is refused here, before anything is queued.  Device allocations that passed are remembered
// per thread by address range, so later calls with the same buffers cost a range lookup.
struct PtrRange {
  uintptr_t lo = 0, hi = 0;
};
thread_local PtrRange t_known[32];
thread_local int t_known_next = 0;

int check_ptr(const void* p, const char* what, const char* who) {
  if (p == nullptr) return kOk;
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  for (const PtrRange& r : t_known)
    if (a >= r.lo && a < r.hi) return kOk;
  hipPointerAttribute_t at;
  const hipError_t e = hipPointerGetAttributes(&at, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // the query's error must not be reported by a later launch check
    return fail(kErrInvalidArg, std::string(who) + ": " + what +
                                    " is not GPU-addressable memory (a host pointer? pass device tensors)");
  }
  if (at.type == hipMemoryTypeHost) return kOk;  // pinned host memory: addressable, not cached here
  if (at.type != hipMemoryTypeDevice && at.type != hipMemoryTypeManaged && at.type != hipMemoryTypeUnified)
    return fail(kErrInvalidArg, std::string(who) + ": " + what +
                                    " is not GPU-addressable memory (a host pointer? pass device tensors)");
  hipDeviceptr_t base = nullptr;
  size_t size = 0;
  if (hipMemGetAddressRange(&base, &size, const_cast<void*>(p)) == hipSuccess && size > 0) {
    PtrRange& r = t_known[t_known_next];
    t_known_next = (t_known_next + 1) % 32;
    r.lo = reinterpret_cast<uintptr_t>(base);
    r.hi = r.lo + size;
  } else {
    (void)hipGetLastError();
  }
  return kOk;
}

struct NamedPtr {
  const void* p;
  const char* name;
};

int check_ptrs(const char* who, std::initializer_list<NamedPtr> ps) {
  for (const NamedPtr& n : ps)
    if (int rc = check_ptr(n.p, n.name, who)) return rc;
  return kOk;
}

int check_linear_ptrs(const char* who, const char* name, const tesm_hip_linear& w) {
  if (int rc = check_ptr(w.packed, name, who)) return rc;
  return check_ptr(w.c_w, name, who);
}

int check_desc_ptrs(const tesm_hip_ent_quant& p) {
  return check_ptrs("local_ent_quant", {{p.q, "q"}, {p.k, "k"}, {p.rope, "rope"}, {p.q_add, "q_add"}, {p.bias, "bias"},
                                        {p.S, "S"}, {p.q_te, "q_te"}, {p.s_te, "s_te"}, {p.rs_te, "rs_te"},
                                        {p.q_c, "q_c"}, {p.s_c, "s_c"}, {p.rs_c, "rs_c"}, {p.e_tanh, "e_tanh"},
                                        {p.c_out, "c_out"}, {p.tern, "tern"}});
}

int check_desc_ptrs(const tesm_hip_output_gate& p) {
  if (int rc = check_ptrs("output_gate", {{p.q_te, "q_te"}, {p.s_te, "s_te"}, {p.rs_te, "rs_te"}, {p.q_c, "q_c"},
                                          {p.s_c, "s_c"}, {p.rs_c, "rs_c"}, {p.local, "local"}, {p.gate, "gate"},
                                          {p.y, "y"}, {p.q_y, "q_y"}, {p.s_y, "s_y"}, {p.rs_y, "rs_y"}}))
    return rc;
  if (int rc = check_linear_ptrs("output_gate", "state_proj", p.state_proj)) return rc;
  return check_linear_ptrs("output_gate", "ent_proj", p.ent_proj);
}

int check_desc_ptrs(const tesm_hip_siso_layer& p) {
  if (int rc = check_ptrs("siso prefill",
                          {{p.u, "u"}, {p.decay_bias, "decay_bias"}, {p.local_bias, "local_bias"}, {p.rope, "rope"},
                           {p.cross_state, "cross_state"}, {p.h0, "h0"}, {p.y, "y"}, {p.states, "states"},
                           {p.h_final, "h_final"}, {p.proj_out, "proj_out"}, {p.k_cache, "k_cache"},
                           {p.v_cache, "v_cache"}, {p.global_embed, "global_embed"}, {p.global_scale, "global_scale"},
                           {p.global_bias, "global_bias"}}))
    return rc;
  for (const auto& w : {std::make_pair(&p.in_proj, "in_proj"), std::make_pair(&p.state_proj, "state_proj"),
                        std::make_pair(&p.ent_proj, "ent_proj"), std::make_pair(&p.out_proj, "out_proj"),
                        std::make_pair(&p.cross_q_proj, "cross_q_proj")})
    if (int rc = check_linear_ptrs("siso prefill", w.second, *w.first)) return rc;
  return kOk;
}

int check_desc_ptrs(const tesm_hip_siso_step& p) {
  if (int rc = check_ptrs("siso decode",
                          {{p.u, "u"}, {p.decay_bias, "decay_bias"}, {p.local_bias, "local_bias"}, {p.rope, "rope"},
                           {p.cross_state, "cross_state"}, {p.state, "state"}, {p.state_out, "state_out"},
                           {p.k_cache, "k_cache"}, {p.v_cache, "v_cache"}, {p.y, "y"}, {p.new_state, "new_state"},
                           {p.step_pos, "step_pos"}}))
    return rc;
  for (const auto& w : {std::make_pair(&p.in_proj, "in_proj"), std::make_pair(&p.state_proj, "state_proj"),
                        std::make_pair(&p.ent_proj, "ent_proj"), std::make_pair(&p.out_proj, "out_proj"),
                        std::make_pair(&p.cross_q_proj, "cross_q_proj")})
    if (int rc = check_linear_ptrs("siso decode", w.second, *w.first)) return rc;
  return kOk;
}

int check_desc_ptrs(const tesm_hip_mimo_layer& p) {
  if (int rc = check_ptrs("mimo prefill",
                          {{p.u, "u"}, {p.decay_bias, "decay_bias"}, {p.local_bias, "local_bias"}, {p.rope, "rope"},
                           {p.mimo_coef, "mimo_coef"}, {p.mimo_x0sq, "mimo_x0sq"}, {p.y, "y"}, {p.h_final, "h_final"},
                           {p.last_state, "last_state"}, {p.k_cache, "k_cache"}, {p.v_cache, "v_cache"},
                           {p.stats_ternary, "stats_ternary"}, {p.stats_counts, "stats_counts"},
                           {p.global_embed, "global_embed"}, {p.global_scale, "global_scale"},
                           {p.global_bias, "global_bias"}}))
    return rc;
  for (const auto& w : {std::make_pair(&p.in_proj, "in_proj"), std::make_pair(&p.state_proj, "state_proj"),
                        std::make_pair(&p.ent_proj, "ent_proj"), std::make_pair(&p.out_proj, "out_proj")})
    if (int rc = check_linear_ptrs("mimo prefill", w.second, *w.first)) return rc;
  return kOk;
}

int check_desc_ptrs(const tesm_hip_mimo_step& p) {
  if (int rc = check_ptrs("mimo decode",
                          {{p.u, "u"}, {p.decay_bias, "decay_bias"}, {p.local_bias, "local_bias"}, {p.rope, "rope"},
                           {p.cross_state, "cross_state"}, {p.state, "state"}, {p.state_out, "state_out"},
                           {p.k_cache, "k_cache"}, {p.v_cache, "v_cache"}, {p.y, "y"}, {p.new_state, "new_state"}}))
    return rc;
  for (const auto& w : {std::make_pair(&p.in_proj, "in_proj"), std::make_pair(&p.state_proj, "state_proj"),
                        std::make_pair(&p.ent_proj, "ent_proj"), std::make_pair(&p.out_proj, "out_proj"),
                        std::make_pair(&p.cross_q_proj, "cross_q_proj")})
    if (int rc = check_linear_ptrs("mimo decode", w.second, *w.first)) return rc;
  return kOk;
}

int check_desc_ptrs(const tesm_hip_rmsnorm& p) {
  return check_ptrs("add_rmsnorm", {{p.x, "x"}, {p.residual, "residual"}, {p.residual_out, "residual_out"},
                                    {p.weight, "weight"}, {p.y, "y"}, {p.q, "q"}, {p.s_x, "s_x"},
                                    {p.rowsum, "rowsum"}});
}

int check_desc_ptrs(const tesm_hip_ffn& p) {
  if (int rc = check_ptrs("ffn", {{p.x, "x"}, {p.x_codes, "x_codes"}, {p.x_scale, "x_scale"},
                                  {p.x_rowsum, "x_rowsum"}, {p.y, "y"}}))
    return rc;
  for (const auto& w : {std::make_pair(&p.gate_proj, "gate_proj"), std::make_pair(&p.up_proj, "up_proj"),
                        std::make_pair(&p.down_proj, "down_proj")})
    if (int rc = check_linear_ptrs("ffn", w.second, *w.first)) return rc;
  return kOk;
}

// Decision taps (tesm_hip_debug_taps): process-wide copy targets for the discrete decisions of
// the layer and step drivers; a driver takes a snapshot when it is called.
std::mutex g_taps_mu;
tesm_hip_taps g_taps{};
bool g_taps_on = false;

bool snapshot_taps(tesm_hip_taps* t) {
  std::lock_guard<std::mutex> g(g_taps_mu);
  *t = g_taps;
  return g_taps_on;
}

int tap_copy(void* dst, const void* src, int64_t bytes, hipStream_t st) {
  if (!dst || !src || bytes <= 0) return kOk;
  if (hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyDeviceToDevice, st) != hipSuccess)
    return fail(kErrLaunch, "decision tap: copy failed");
  return kOk;
}

int tap_codes(int8_t* q, float* sc, const CodeBuf& b, int64_t M, hipStream_t st) {
  if (int rc = tap_copy(q, b.q, M * b.ldq, st)) return rc;
  return tap_copy(sc, b.s, M * 4, st);
}

// Workspace layout of the SISO prefill; with base == nullptr it only measures.
struct SisoPlan {
  bool fuse_ent;  // entanglement kernel also quantizes tanh(E) and C
  bool rowq;      // output gate kernel also quantizes y (d_model <= 1024)
  CodeBuf xu, xe, xc, xy, xs;
  void* proj;
  void* scan_ws;
  int64_t scan_bytes;
  float* wts;
  void* e_tanh;
  void* c_mix;
  void* yg;
  void* cq;
  int8_t* g_tern;   // global entanglement (window == 0): decisions, counts, bias table, RoPE'd q / k,
  int32_t* g_count; // bf16 states transposed
  uint16_t* g_st;
  float* g_table;
  float *g_qr, *g_kr;
  int64_t total;
};

EntArgs siso_ent_shape(const tesm_hip_siso_layer& p) {
  EntArgs e;
  e.dt = p.dt;
  e.mimo = 0;
  e.B = p.B;
  e.L = p.L;
  e.H = 1;
  e.R = p.ent_rank;
  e.D = p.d_state;
  e.W = p.window;
  e.ldq = kpad(p.d_state);
  return e;
}

SisoPlan plan_siso(const tesm_hip_siso_layer& p, void* base) {
  Carve c(base);
  SisoPlan s;
  const int64_t M = p.B * p.L;
  const int64_t n_in = 2 * p.d_model + 3 * p.d_state + 2 * p.ent_rank;
  const int es = esize(p.dt);
  const bool global = p.window == 0;
  s.fuse_ent = !global && ent_fused_ok(siso_ent_shape(p));
  // the row-complete gate keeps both weight matrices in LDS, one workgroup per CU streaming 16-row
  // tiles: it pays with many tiles; short prefills (fewer than 256 tiles) take the tiled gate
  s.rowq = p.d_model <= 1024 && M >= 4096;
  s.xu = take_codes(c, M, p.d_model);
  s.proj = c.take<void>(M * n_in * es);
  s.scan_bytes = scan_ws_bytes(p.B, p.L, p.d_state, p.chunk_size);
  s.scan_ws = c.take<void>(s.scan_bytes);
  s.wts = nullptr;
  s.e_tanh = s.c_mix = nullptr;
  s.g_tern = nullptr;
  s.g_count = nullptr;
  s.g_st = nullptr;
  s.g_table = nullptr;
  s.g_qr = s.g_kr = nullptr;
  if (!s.fuse_ent) {
    if (global) {
      s.g_tern = c.take<int8_t>(p.B * p.L * global_tern_pitch(p.L));
      s.g_count = c.take<int32_t>(p.B * p.L * 4);
      s.g_table = c.take<float>(2 * p.L * 4);
      s.g_qr = c.take<float>(p.B * p.L * p.ent_rank * 4);
      s.g_kr = c.take<float>(p.B * p.L * p.ent_rank * 4);
      s.g_st = p.dt == kBF16 ? c.take<uint16_t>(global_states_t_bytes(p.dt, 0, p.B, p.L, p.d_state)) : nullptr;
    } else {
      s.wts = c.take<float>(ent_ws_bytes(p.B, p.L, 1, std::min(p.window, p.L)));
    }
    s.e_tanh = c.take<void>(M * p.d_state * es);
    s.c_mix = c.take<void>(M * p.d_state * es);
  }
  s.xe = take_codes(c, M, p.d_state);
  s.xc = take_codes(c, M, p.d_state);
  s.yg = s.rowq ? nullptr : c.take<void>(M * p.d_model * es);
  s.xy = take_codes(c, M, p.d_model);
  if (p.cross_state) {
    s.xs = take_codes(c, M, p.d_state);
    s.cq = c.take<void>(M * p.ent_rank * es);
  } else {
    s.xs = CodeBuf{nullptr, nullptr, nullptr, 0};
    s.cq = nullptr;
  }
  s.total = c.off;
  return s;
}

int check_linear(const tesm_hip_linear& w, int64_t K, const char* name) {
  TESM_REQUIRE(w.packed && w.c_w, kErrInvalidArg, std::string("siso layer: null ") + name);
  TESM_REQUIRE(w.ldw >= kpad(K) / 4 && w.ldw % 16 == 0, kErrInvalidArg,
               std::string("siso layer: ") + name + " ldw must be >= kpad(K)/4 and a multiple of 16");
  return kOk;
}

int run_linear(const CodeBuf& x, const tesm_hip_linear& w, int64_t M, int64_t N, int64_t K, void* out, int dt,
               int64_t ldo, hipStream_t st) {
  LinearArgs a;
  a.op[0] = operand(x, w);
  a.M = M;
  a.N = N;
  a.Kp = kpad(K);
  a.out = out;
  a.out_dt = dt;
  a.ldo = ldo;
  return launch_linear(a, st);
}

// state_proj(tanh E), ent_proj(C) and the output gate y = local + sigmoid(gate) * sp + ep
// (tesm.py:1256-1260), quantized per token for out_proj, then out_proj (tesm.py:1261; dropout is
// identity in eval).  Rows: M; local / gate are column slices of the in_proj output.
struct OutputPath {
  CodeBuf xe, xc, xy;
  void* yg;  // (M, d_model) scratch for the tiled gate when the row-complete kernel cannot run
  const tesm_hip_linear *state_proj, *ent_proj, *out_proj;
  int64_t M, dm, D;
  int dt;
  float eps;
  const void* local;
  const void* gate;
  int64_t ld;
  void* y;
  const tesm_hip_taps* taps = nullptr;  // set: copy out y's codes (quantized apart from out_proj)
};

int run_output_path(const OutputPath& o, hipStream_t st) {
  LinearArgs ga;
  ga.op[0] = operand(o.xe, *o.state_proj);
  ga.op[1] = operand(o.xc, *o.ent_proj);
  ga.M = o.M;
  ga.N = o.dm;
  ga.Kp = kpad(o.D);
  ga.out_dt = o.dt;
  ga.epilogue = kEpiOutputGate;
  ga.local = o.local;
  ga.ld_local = o.ld;
  ga.gate = o.gate;
  ga.ld_gate = o.ld;
  int rc;
  if (!o.yg) {
    RowQuant rq;
    rq.q = o.xy.q;
    rq.ldq = o.xy.ldq;
    rq.s = o.xy.s;
    rq.rs = o.xy.rs;
    rq.eps = o.eps;
    if (o.taps && o.taps->yv) {  // the row-complete gate also writes y itself
      rq.y = o.taps->yv;
      rq.ldy = o.dm;
    }
    // the gate and out_proj in one launch where the 32-row kernel takes both: y's codes stay in LDS
    // (written out only for the decision taps).  TESM_HIP_NO_GATE_OUT=1 keeps the two launches (a
    // diagnostic switch, read per call: the results are the same bits)
    const char* no_fuse = std::getenv("TESM_HIP_NO_GATE_OUT");
    if (!(no_fuse && no_fuse[0] == '1')) {
      RowQuant rf = rq;
      if (!o.taps) {
        rf.q = nullptr;
        rf.s = nullptr;
        rf.rs = nullptr;
      }
      rc = launch_gate_out(ga, rf, operand(o.xy, *o.out_proj), o.y, o.dm, st);
      if (rc == kOk) {
        if (o.taps && (rc = tap_codes(o.taps->q_y, o.taps->s_y, o.xy, o.M, st))) return rc;
        return kOk;
      }
      if (rc > 0) return rc;
    }
    if ((rc = launch_gate_rowq(ga, rq, st))) return rc;
    if (o.taps && (rc = tap_codes(o.taps->q_y, o.taps->s_y, o.xy, o.M, st))) return rc;
  } else {
    ga.out = o.yg;
    ga.ldo = o.dm;
    if ((rc = launch_linear(ga, st))) return rc;
    LinearArgs la;
    la.op[0] = operand(o.xy, *o.out_proj);
    la.M = o.M;
    la.N = o.dm;
    la.Kp = kpad(o.dm);
    la.out = o.y;
    la.out_dt = o.dt;
    la.ldo = o.dm;
    if (!o.taps && linear_fq_ok(la)) {  // decode-size batches: y's quantization inside out_proj, one launch fewer
      FusedQuantIn f;
      f.x = o.yg;
      f.ldx = o.dm;
      f.K = o.dm;
      f.eps = o.eps;
      f.dt = o.dt;
      return launch_linear_fq(la, f, st);
    }
    if ((rc = launch_quant_act(o.yg, o.dt, o.M, o.dm, o.dm, o.eps, 1, o.xy.q, o.xy.ldq, o.xy.s, o.xy.rs, st)))
      return rc;
    if (o.taps && (rc = tap_codes(o.taps->q_y, o.taps->s_y, o.xy, o.M, st))) return rc;
    if (o.taps && (rc = tap_copy(o.taps->yv, o.yg, o.M * o.dm * esize(o.dt), st))) return rc;
    return launch_linear(la, st);
  }
  return run_linear(o.xy, *o.out_proj, o.M, o.dm, o.dm, o.y, o.dt, o.dm, st);
}

// Workspace layout of the SISO decode step; with base == nullptr it only measures.
struct DecodePlan {
  CodeBuf xu, xs, xe, xc, xy;
  void* proj;
  void* cq;
  void* yg;
  int64_t total;
};

DecodePlan plan_decode(const tesm_hip_siso_step& p, void* base) {
  Carve c(base);
  DecodePlan s;
  const int64_t n_in = 2 * p.d_model + 3 * p.d_state + 2 * p.ent_rank;
  const int es = esize(p.dt);
  s.xu = take_codes(c, p.B, p.d_model);
  s.proj = c.take<void>(p.B * n_in * es);
  if (p.cross_state) {
    s.xs = take_codes(c, p.B, p.d_state);
    s.cq = c.take<void>(p.B * p.ent_rank * es);
  } else {
    s.xs = CodeBuf{nullptr, nullptr, nullptr, 0};
    s.cq = nullptr;
  }
  s.xe = take_codes(c, p.B, p.d_state);
  s.xc = take_codes(c, p.B, p.d_state);
  // the row-complete gate stages both weight matrices in LDS per workgroup, which only pays with
  // many 16-row tiles; a decode batch takes the tiled gate and a separate quantization (same values)
  s.yg = p.d_model <= 1024 && p.B >= 256 ? nullptr : c.take<void>(p.B * p.d_model * es);
  s.xy = take_codes(c, p.B, p.d_model);
  s.total = c.off;
  return s;
}

// Workspace layout of the MIMO prefill; with base == nullptr it only measures.
struct MimoPlan {
  CodeBuf xu, xe, xc, xy;
  void* proj;
  void* scan_ws;
  int64_t scan_bytes;
  float* S;
  float* wts;
  void* te;
  void* cc;
  void* yg;
  int8_t* g_tern;  // global entanglement (window == 0)
  int32_t* g_count;
  float* g_table;
  float *g_qr, *g_kr;
  int64_t total;
};

// Thread-chunk length of the MIMO state scan.  Its recurrence has no clamp (tesm_mimo.py:375-392 is
// the plain sequential h = d h + u), so the chunk only sets the scan's work split: 32 positions per
// wave halve the look-back spans of 16 (configs[4]: 0.52 against 0.65 ms).
constexpr int64_t kMimoScanChunk = 32;

MimoPlan plan_mimo(const tesm_hip_mimo_layer& p, void* base) {
  Carve c(base);
  MimoPlan s;
  const int64_t M = p.B * p.L, HD = p.n_heads * p.d_state;
  const int64_t n_in = 2 * p.d_model + 3 * HD + 2 * p.n_heads * p.ent_rank;
  const int es = esize(p.dt);
  s.xu = take_codes(c, M, p.d_model);
  s.proj = c.take<void>(M * n_in * es);
  s.scan_bytes = scan_ws_bytes(p.B, p.L, HD, kMimoScanChunk);
  s.scan_ws = c.take<void>(s.scan_bytes);
  s.S = c.take<float>(M * HD * 4);
  s.wts = nullptr;
  s.g_tern = nullptr;
  s.g_count = nullptr;
  s.g_table = nullptr;
  s.g_qr = s.g_kr = nullptr;
  if (p.window > 0) {
    s.wts = c.take<float>(ent_ws_bytes(p.B, p.L, p.n_heads, p.window));
  } else {
    s.g_tern = c.take<int8_t>(p.B * p.L * global_tern_pitch(p.L));
    s.g_count = c.take<int32_t>(p.B * p.L * 4);
    s.g_table = c.take<float>(2 * p.L * 4);
    s.g_qr = c.take<float>(p.B * p.L * p.n_heads * p.ent_rank * 4);
    s.g_kr = c.take<float>(p.B * p.L * p.n_heads * p.ent_rank * 4);
  }
  s.te = c.take<void>(M * HD * es);
  s.cc = c.take<void>(M * HD * es);
  s.xe = take_codes(c, M, HD);
  s.xc = take_codes(c, M, HD);
  s.yg = p.d_model <= 1024 && M >= 4096 ? nullptr : c.take<void>(M * p.d_model * es);
  s.xy = take_codes(c, M, p.d_model);
  s.total = c.off;
  return s;
}

// Workspace layout of the feed-forward; with base == nullptr it only measures.
struct FfnPlan {
  CodeBuf xq, hq;
  void* h;
  int64_t total;
};

FfnPlan plan_ffn(const tesm_hip_ffn& p, void* base) {
  Carve c(base);
  FfnPlan s;
  if (p.x_codes)
    s.xq = CodeBuf{nullptr, nullptr, nullptr, 0};
  else
    s.xq = take_codes(c, p.M, p.d_model);
  s.h = c.take<void>(p.M * p.d_inter * esize(p.dt));
  s.hq = take_codes(c, p.M, p.d_inter);
  s.total = c.off;
  return s;
}

}  // namespace

// Scratch memory of the allocation-free decode entry point (tesm_hip_siso_decode_noalloc): one
// array per device, held until the process ends.  Host code never passes the array's name to a
// kernel (in host code it is only a stand-in for the symbol): it uses the device address that
// hipGetSymbolAddress returns, looked up once per device.
constexpr int64_t kNoAllocScratchBytes = TESM_HIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};

// The current device's scratch address (nullptr and an error message if it cannot be found).
void* scratch_ptr() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    set_error("no-alloc decode: no current device (or more than 64 devices)");
    return nullptr;
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      set_error(std::string("no-alloc decode: hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}
}  // namespace
}  // namespace tesm

using namespace tesm;

extern "C" {

int tesm_hip_abi_version(void) { return TESM_HIP_ABI_VERSION; }

int tesm_hip_launch_log(int enable) {
  std::lock_guard<std::mutex> g(g_log_mu);
  g_log.clear();
  __atomic_store_n(&g_launch_log_on, enable ? 1 : 0, __ATOMIC_RELAXED);
  return kOk;
}

int tesm_hip_stream_copy(void* dst, const void* src, int64_t bytes, void* stream) {
  if (int rc = check_ptrs("stream copy", {{dst, "dst"}, {src, "src"}})) return rc;
  return launch_stream_copy(dst, src, bytes, static_cast<hipStream_t>(stream));
}

int tesm_hip_device_status(uint32_t* status, int clear) {
  unsigned v = 0;
  if (int rc = scan_status(&v, clear)) return rc;
  if (status) *status = v;
  return kOk;
}

int tesm_hip_debug_taps(const tesm_hip_taps* t) {
  std::lock_guard<std::mutex> g(g_taps_mu);
  g_taps_on = t != nullptr;
  g_taps = t ? *t : tesm_hip_taps{};
  return kOk;
}

int tesm_hip_debug_scan_spin_limit(int limit) {
  scan_set_spin_limit(limit);
  return kOk;
}

int64_t tesm_hip_launch_log_read(char* buf, int64_t cap, int clear) {
  std::lock_guard<std::mutex> g(g_log_mu);
  const int64_t n = static_cast<int64_t>(g_log.size());
  if (buf && cap > 0) {
    const int64_t k = std::min<int64_t>(n, cap - 1);
    std::memcpy(buf, g_log.data(), static_cast<size_t>(k));
    buf[k] = '\0';
  }
  if (clear) g_log.clear();
  return n;
}

const char* tesm_hip_last_error(void) { return g_last_error.c_str(); }

int64_t tesm_hip_kpad(int64_t K) { return kpad(K); }

int tesm_hip_quant_act_i8(const void* x, int dt, int64_t M, int64_t K, int64_t ldx, float eps, int layout, int8_t* q,
                          int64_t ldq, float* s_x, int32_t* rowsum, void* stream) {
  if (int rc = check_ptrs("quant_act", {{x, "x"}, {q, "q"}, {s_x, "s_x"}, {rowsum, "rowsum"}})) return rc;
  return launch_quant_act(x, dt, M, K, ldx, eps, layout, q, ldq, s_x, rowsum, static_cast<hipStream_t>(stream));
}

int64_t tesm_hip_absmean_ws_bytes(void) { return 512 * static_cast<int64_t>(sizeof(double)); }

int tesm_hip_absmean_scale(const void* w, int dt, int64_t n, float eps, void* ws, float* s_w, float* c_w,
                           void* stream) {
  if (int rc = check_ptrs("absmean", {{w, "w"}, {ws, "ws"}, {s_w, "s_w"}, {c_w, "c_w"}})) return rc;
  return launch_absmean(w, dt, n, eps, static_cast<double*>(ws), s_w, c_w, static_cast<hipStream_t>(stream));
}

int tesm_hip_pack_w_i2(const void* w, int dt, int64_t N, int64_t K, int64_t ldw, const float* s_w, int per_row,
                       uint8_t* packed, int64_t ldp, void* stream) {
  if (int rc = check_ptrs("pack_w_i2", {{w, "w"}, {s_w, "s_w"}, {packed, "packed"}})) return rc;
  return launch_pack(w, dt, N, K, ldw, s_w, per_row, packed, ldp, static_cast<hipStream_t>(stream));
}

int tesm_hip_unpack_w_i2(const uint8_t* packed, int64_t N, int64_t K, int64_t ldp, int8_t* codes, int64_t ldc,
                         void* stream) {
  if (int rc = check_ptrs("unpack_w_i2", {{packed, "packed"}, {codes, "codes"}})) return rc;
  return launch_unpack(packed, N, K, ldp, codes, ldc, static_cast<hipStream_t>(stream));
}

int tesm_hip_bitlinear_i2(const int8_t* q, int64_t ldq, const float* s_x, const int32_t* rowsum,
                          const uint8_t* packed, int64_t ldw, const float* c_w, int c_w_per_row, const void* bias,
                          int64_t M, int64_t N, int64_t K, void* out, int out_dt, int64_t ldo, int32_t* acc_dump,
                          void* stream) {
  if (int rc = check_ptrs("bitlinear", {{q, "q"}, {s_x, "s_x"}, {rowsum, "rowsum"}, {packed, "packed"}, {c_w, "c_w"},
                                         {bias, "bias"}, {out, "out"}, {acc_dump, "acc_dump"}}))
    return rc;
  TESM_REQUIRE(K >= 1, kErrInvalidArg, "bitlinear: K must be >= 1");
  LinearArgs a;
  a.op[0].q = q;
  a.op[0].ldq = ldq;
  a.op[0].s_x = s_x;
  a.op[0].rowsum = rowsum;
  a.op[0].w = packed;
  a.op[0].ldw = ldw;
  a.op[0].c_w = c_w;
  a.op[0].c_w_per_row = c_w_per_row;
  a.M = M;
  a.N = N;
  a.Kp = kpad(K);
  a.bias = bias;
  a.out = out;
  a.out_dt = out_dt;
  a.ldo = ldo;
  a.acc_dump = acc_dump;
  return launch_linear(a, static_cast<hipStream_t>(stream));
}

int64_t tesm_hip_bitlinear_fwd_ws_bytes(int64_t M, int64_t K) {
  Carve c(nullptr);
  take_codes(c, std::max<int64_t>(M, 1), K);
  return c.off;
}

int tesm_hip_bitlinear_fwd(const void* x, int dt, int64_t ldx, float eps, const uint8_t* packed, int64_t ldw,
                           const float* c_w, int c_w_per_row, const void* bias, int64_t M, int64_t N, int64_t K,
                           void* out, int out_dt, int64_t ldo, int fuse, void* ws, int64_t ws_bytes, void* stream) {
  if (int rc = check_ptrs("bitlinear fwd", {{x, "x"}, {packed, "packed"}, {c_w, "c_w"}, {bias, "bias"}, {out, "out"},
                                            {ws, "ws"}}))
    return rc;
  TESM_REQUIRE(K >= 1 && M >= 0 && N >= 0, kErrInvalidArg, "bitlinear fwd: bad sizes");
  TESM_REQUIRE(dt == kF32 || dt == kBF16, kErrInvalidArg, "bitlinear fwd: x dtype must be 0 or 1");
  TESM_REQUIRE(ldx >= K, kErrInvalidArg, "bitlinear fwd: ldx must be >= K");
  if (M == 0 || N == 0) return kOk;
  hipStream_t st = static_cast<hipStream_t>(stream);
  LinearArgs la;
  la.op[0].w = packed;
  la.op[0].ldw = ldw;
  la.op[0].c_w = c_w;
  la.op[0].c_w_per_row = c_w_per_row;
  la.M = M;
  la.N = N;
  la.Kp = kpad(K);
  la.bias = bias;
  la.out = out;
  la.out_dt = out_dt;
  la.ldo = ldo;
  if (fuse && linear_fq_ok(la)) {
    FusedQuantIn f;
    f.x = x;
    f.ldx = ldx;
    f.K = K;
    f.eps = eps;
    f.dt = dt;
    return launch_linear_fq(la, f, st);
  }
  Carve c(ws);
  const CodeBuf cb = take_codes(c, M, K);
  TESM_REQUIRE(ws && ws_bytes >= c.off, kErrWorkspace, "bitlinear fwd: workspace too small");
  if (int rc = launch_quant_act(x, dt, M, K, ldx, eps, 1, cb.q, cb.ldq, cb.s, cb.rs, st)) return rc;
  la.op[0].q = cb.q;
  la.op[0].ldq = cb.ldq;
  la.op[0].s_x = cb.s;
  la.op[0].rowsum = cb.rs;
  return launch_linear(la, st);
}

int64_t tesm_hip_scan_ws_bytes(int64_t B, int64_t L, int64_t C, int64_t chunk_size) {
  return scan_ws_bytes(B, L, C, chunk_size);
}

int tesm_hip_scan(const void* decay, int64_t ld_decay, const void* update, int64_t ld_update, int dt, int64_t B,
                  int64_t L, int64_t C, int64_t chunk_size, const double* h0, void* states, int64_t ld_states,
                  int out_dt, double* h_final, void* ws, int64_t ws_bytes, void* stream) {
  if (int rc = check_ptrs("scan", {{decay, "decay"}, {update, "update"}, {h0, "h0"}, {states, "states"},
                                    {h_final, "h_final"}, {ws, "ws"}}))
    return rc;
  ScanArgs a;
  a.mode = 0;
  a.dt = dt;
  a.out_dt = out_dt;
  a.clamp = 1;
  a.B = B;
  a.L = L;
  a.C = C;
  a.cs = chunk_size;
  a.decay = decay;
  a.ld_decay = ld_decay;
  a.update = update;
  a.ld_update = ld_update;
  a.h0 = h0;
  a.states = states;
  a.ld_states = ld_states;
  a.h_final = h_final;
  return launch_scan(a, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

int tesm_hip_rope_table(void* tab, int64_t L, int64_t R, int64_t pos_offset, double base, int dt, void* stream) {
  if (int rc = check_ptrs("rope_table", {{tab, "tab"}})) return rc;
  return launch_rope_table(static_cast<float2*>(tab), L, R, pos_offset, base, dt, static_cast<hipStream_t>(stream));
}

int64_t tesm_hip_local_ent_ws_bytes(int64_t B, int64_t L, int64_t H, int64_t W) { return ent_ws_bytes(B, L, H, W); }

int tesm_hip_local_ent(const void* q, int64_t ld_q, const void* k, int64_t ld_k, const void* rope, const void* q_add,
                       int64_t ld_qadd, const float* bias, const void* S, int64_t ld_s, int dt, int mimo, int64_t B,
                       int64_t L, int64_t H, int64_t R, int64_t D, int64_t W, float thr, float ent_scale, void* avg,
                       void* e_out, void* c_out, void* e_tanh, int64_t ld_out, int8_t* tern, void* ws,
                       int64_t ws_bytes, void* stream) {
  if (int rc = check_ptrs("local_ent", {{q, "q"}, {k, "k"}, {rope, "rope"}, {q_add, "q_add"}, {bias, "bias"}, {S, "S"},
                                         {avg, "avg"}, {e_out, "e_out"}, {c_out, "c_out"}, {e_tanh, "e_tanh"},
                                         {tern, "tern"}, {ws, "ws"}}))
    return rc;
  EntArgs a;
  a.dt = dt;
  a.mimo = mimo;
  a.B = B;
  a.L = L;
  a.H = H;
  a.R = R;
  a.D = D;
  a.W = W;
  a.q = q;
  a.ld_q = ld_q;
  a.k = k;
  a.ld_k = ld_k;
  a.rope = static_cast<const float2*>(rope);
  a.q_add = q_add;
  a.ld_qadd = ld_qadd;
  a.bias = bias;
  a.thr = thr;
  a.ent_scale = ent_scale;
  a.S = S;
  a.ld_s = ld_s;
  a.avg = avg;
  a.e_out = e_out;
  a.c_out = c_out;
  a.e_tanh = e_tanh;
  a.ld_out = ld_out;
  a.tern = tern;
  a.wts = static_cast<float*>(ws);
  const int64_t weff = mimo ? W : std::min(W, L);
  TESM_REQUIRE(ws && ws_bytes >= ent_ws_bytes(B, L, H, weff), kErrWorkspace, "local_ent: workspace too small");
  return launch_local_ent(a, static_cast<hipStream_t>(stream));
}

int tesm_hip_local_ent_quant(const tesm_hip_ent_quant* p, void* stream) {
  TESM_REQUIRE(p != nullptr, kErrInvalidArg, "local_ent_quant: null descriptor");
  if (int rc = check_desc_ptrs(*p)) return rc;
  EntArgs a;
  a.dt = p->dt;
  a.mimo = 0;
  a.B = p->B;
  a.L = p->L;
  a.H = 1;
  a.R = p->R;
  a.D = p->D;
  a.W = p->W;
  a.q = p->q;
  a.ld_q = p->ld_q;
  a.k = p->k;
  a.ld_k = p->ld_k;
  a.rope = static_cast<const float2*>(p->rope);
  a.q_add = p->q_add;
  a.ld_qadd = p->ld_qadd;
  a.bias = p->bias;
  a.thr = p->thr;
  a.ent_scale = p->ent_scale;
  a.S = p->S;
  a.ld_s = p->ld_s;
  a.e_tanh = p->e_tanh;
  a.c_out = p->c_out;
  a.ld_out = p->ld_out;
  a.tern = p->tern;
  a.q_te = p->q_te;
  a.s_te = p->s_te;
  a.rs_te = p->rs_te;
  a.q_c = p->q_c;
  a.s_c = p->s_c;
  a.rs_c = p->rs_c;
  a.ldq = p->ldq;
  a.eps = p->eps;
  TESM_REQUIRE(a.q_te != nullptr, kErrInvalidArg, "local_ent_quant: q_te is required");
  return launch_local_ent(a, static_cast<hipStream_t>(stream));
}

int tesm_hip_output_gate_i2(const tesm_hip_output_gate* p, void* stream) {
  TESM_REQUIRE(p != nullptr, kErrInvalidArg, "output_gate: null descriptor");
  if (int rc = check_desc_ptrs(*p)) return rc;
  CodeBuf te{const_cast<int8_t*>(p->q_te), const_cast<float*>(p->s_te), const_cast<int32_t*>(p->rs_te), p->ldq_te};
  CodeBuf cc{const_cast<int8_t*>(p->q_c), const_cast<float*>(p->s_c), const_cast<int32_t*>(p->rs_c), p->ldq_c};
  LinearArgs ga;
  ga.op[0] = operand(te, p->state_proj);
  ga.op[1] = operand(cc, p->ent_proj);
  ga.M = p->M;
  ga.N = p->d_model;
  ga.Kp = kpad(p->d_state);
  ga.out_dt = p->dt;
  ga.epilogue = kEpiOutputGate;
  ga.local = p->local;
  ga.ld_local = p->ld_local;
  ga.gate = p->gate;
  ga.ld_gate = p->ld_gate;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (p->q_y) {
    RowQuant rq;
    rq.q = p->q_y;
    rq.ldq = p->ldq_y;
    rq.s = p->s_y;
    rq.rs = p->rs_y;
    rq.eps = p->eps;
    rq.y = p->y;
    rq.ldy = p->ld_y;
    return launch_gate_rowq(ga, rq, st);
  }
  TESM_REQUIRE(p->y != nullptr, kErrInvalidArg, "output_gate: need y or q_y");
  ga.out = p->y;
  ga.ldo = p->ld_y;
  return launch_linear(ga, st);
}

int64_t tesm_hip_siso_prefill_ws_bytes(const tesm_hip_siso_layer* p) {
  if (!p) return -1;
  return plan_siso(*p, nullptr).total;
}

int tesm_hip_siso_prefill(const tesm_hip_siso_layer* pp, void* ws, int64_t ws_bytes, void* stream) {
  TESM_REQUIRE(pp != nullptr, kErrInvalidArg, "siso layer: null descriptor");
  if (int rc = check_desc_ptrs(*pp)) return rc;
  const tesm_hip_siso_layer& p = *pp;
  hipStream_t st = static_cast<hipStream_t>(stream);
  TESM_REQUIRE(p.dt == kF32 || p.dt == kBF16, kErrInvalidArg, "siso layer: dtype must be 0 or 1");
  TESM_REQUIRE(p.B >= 1 && p.L >= 1 && p.d_model >= 1 && p.d_state >= 1 && p.ent_rank >= 2 && p.ent_rank % 2 == 0 &&
                   p.window >= 0 && p.window <= 64 && p.chunk_size >= 1,
               kErrInvalidArg, "siso layer: bad sizes (need even ent_rank, 0 <= window <= 64)");
  TESM_REQUIRE(p.u && p.decay_bias && (p.local_bias || p.window == 0) && p.rope && p.y && p.states, kErrInvalidArg,
               "siso layer: null pointer");
  TESM_REQUIRE(p.window > 0 || (p.global_embed && p.global_dim >= 1 && p.global_scale && p.global_bias),
               kErrInvalidArg, "siso layer: global entanglement (window 0) needs the relative-position parameters");
  TESM_REQUIRE(p.cache_window >= 0 && (p.window > 0 || p.cache_window > 0 || !(p.k_cache || p.v_cache)),
               kErrInvalidArg, "siso layer: a cache with window 0 needs cache_window");
  if (int rc = check_linear(p.in_proj, p.d_model, "in_proj")) return rc;
  if (int rc = check_linear(p.state_proj, p.d_state, "state_proj")) return rc;
  if (int rc = check_linear(p.ent_proj, p.d_state, "ent_proj")) return rc;
  if (int rc = check_linear(p.out_proj, p.d_model, "out_proj")) return rc;
  if (p.cross_state)
    if (int rc = check_linear(p.cross_q_proj, p.d_state, "cross_q_proj")) return rc;
  const SisoPlan s = plan_siso(p, ws);
  TESM_REQUIRE(ws && ws_bytes >= s.total, kErrWorkspace, "siso layer: workspace too small");
  tesm_hip_taps tp;
  const bool tapping = snapshot_taps(&tp);

  const int dt = p.dt;
  const int es = esize(dt);
  const int64_t M = p.B * p.L, dm = p.d_model, D = p.d_state, R = p.ent_rank;
  const int64_t n_in = 2 * dm + 3 * D + 2 * R;
  char* proj = static_cast<char*>(s.proj);
  // slice offsets of the in_proj output (tesm.py:1197-1201)
  const int64_t o_local = 0, o_sv = dm, o_decay = dm + D, o_write = dm + 2 * D, o_gate = dm + 3 * D,
                o_q = 2 * dm + 3 * D, o_k = 2 * dm + 3 * D + R;
  int rc;
  // 1. in_proj
  // the u quantization also clears the single-pass scan's flags, saving the scan its reset launch
  int* scan_zero = nullptr;
  int64_t scan_zero_n = 0;
  scan_lb_clear_range(p.B, p.L, D, p.chunk_size, s.scan_ws, &scan_zero, &scan_zero_n);
  if ((rc = launch_quant_act(p.u, dt, M, dm, dm, p.bit_eps, 1, s.xu.q, s.xu.ldq, s.xu.s, s.xu.rs, st, scan_zero,
                             scan_zero_n)))
    return rc;
  if (tapping && (rc = tap_codes(tp.q_u, tp.s_u, s.xu, M, st))) return rc;
  // (the scan applies the gates: at K = d_model 768 an in_proj epilogue that applies them, as the MIMO
  // prefill's does, costs the product 4.3 us and saves the scan 2.6 us)
  if ((rc = run_linear(s.xu, p.in_proj, M, n_in, dm, proj, dt, n_in, st))) return rc;
  if (p.proj_out) {
    if (hipMemcpyAsync(p.proj_out, proj, M * n_in * es, hipMemcpyDeviceToDevice, st) != hipSuccess)
      return fail(kErrLaunch, "siso layer: proj copy failed");
  }
  // 2. cross-layer query bias (tesm.py:1213-1218)
  if (p.cross_state) {
    if ((rc = launch_quant_act(p.cross_state, dt, M, D, D, p.bit_eps, 1, s.xs.q, s.xs.ldq, s.xs.s, s.xs.rs, st)))
      return rc;
    if (tapping && (rc = tap_codes(tp.q_cs, tp.s_cs, s.xs, M, st))) return rc;
    if ((rc = run_linear(s.xs, p.cross_q_proj, M, R, D, s.cq, dt, R, st))) return rc;
  }
  // 3. gates + state scan (tesm.py:1202-1205, 1222-1223)
  ScanArgs sa;
  sa.mode = 1;
  sa.dt = dt;
  sa.out_dt = dt;
  sa.clamp = 1;
  sa.round_update = 1;
  sa.B = p.B;
  sa.L = p.L;
  sa.C = D;
  sa.cs = p.chunk_size;
  sa.decay = proj + o_decay * es;
  sa.ld_decay = n_in;
  sa.update = proj + o_write * es;
  sa.ld_update = n_in;
  sa.sv = proj + o_sv * es;
  sa.ld_sv = n_in;
  sa.decay_bias = p.decay_bias;
  sa.h0 = p.h0;
  sa.states = p.states;
  sa.ld_states = D;
  sa.h_final = p.h_final;
  sa.flags_clear = scan_zero_n > 0;
  if ((rc = launch_scan(sa, s.scan_ws, s.scan_bytes, st))) return rc;
  // 4. local entanglement + mix (tesm.py:853-952, 1231-1232), quantized for state_proj / ent_proj
  EntArgs ea = siso_ent_shape(p);
  ea.q = proj + o_q * es;
  ea.ld_q = n_in;
  ea.k = proj + o_k * es;
  ea.ld_k = n_in;
  ea.rope = static_cast<const float2*>(p.rope);
  ea.q_add = s.cq;
  ea.ld_qadd = R;
  ea.bias = p.local_bias;
  ea.thr = p.thr;
  ea.ent_scale = p.ent_scale;
  ea.S = p.states;
  ea.ld_s = D;
  ea.eps = p.bit_eps;
  if (tapping) ea.tern = tp.tern;
  if (p.window == 0) {  // global causal entanglement (tesm.py:963-1063), then the same quantizations
    if ((rc = launch_global_bias_table(dt, 2 * p.L, p.global_embed, p.global_dim, p.global_scale, p.global_bias,
                                       s.g_table, st)))
      return rc;
    GlobalArgs ga;
    ga.dt = dt;
    ga.mimo = 0;
    ga.B = p.B;
    ga.L = p.L;
    ga.H = 1;
    ga.R = R;
    ga.D = D;
    ga.q = ea.q;
    ga.ld_q = n_in;
    ga.k = ea.k;
    ga.ld_k = n_in;
    ga.rope = ea.rope;
    ga.q_add = s.cq;
    ga.ld_qadd = R;
    ga.table = s.g_table;
    ga.thr = p.thr;
    ga.sqrt_div = static_cast<float>(std::sqrt(static_cast<double>(R)));
    ga.ent_scale = p.ent_scale;
    ga.S = p.states;
    ga.ld_s = D;
    ga.e_tanh = s.e_tanh;
    ga.c_out = s.c_mix;
    ga.ld_out = D;
    ga.tern = s.g_tern;
    ga.count = s.g_count;
    ga.states_t = s.g_st;
    ga.qr = s.g_qr;
    ga.kr = s.g_kr;
    if ((rc = launch_global_ent(ga, st))) return rc;
    if (tapping && (rc = tap_copy(tp.tern, s.g_tern, M * global_tern_pitch(p.L), st))) return rc;
    if (tapping && (rc = tap_copy(tp.te, s.e_tanh, M * D * es, st))) return rc;
    if (tapping && (rc = tap_copy(tp.c, s.c_mix, M * D * es, st))) return rc;
    if ((rc = quant_te_c(s.e_tanh, s.c_mix, dt, M, D, p.bit_eps, s.xe, s.xc, st))) return rc;
  } else if (s.fuse_ent) {
    ea.q_te = s.xe.q;
    ea.s_te = s.xe.s;
    ea.rs_te = s.xe.rs;
    ea.q_c = s.xc.q;
    ea.s_c = s.xc.s;
    ea.rs_c = s.xc.rs;
    ea.ldq = s.xe.ldq;
    if (tapping && tp.te && tp.c) {  // the fused kernel also writes the float values it quantizes
      ea.e_tanh = tp.te;
      ea.c_out = tp.c;
      ea.ld_out = D;
    }
    if ((rc = launch_local_ent(ea, st))) return rc;
  } else {
    ea.e_tanh = s.e_tanh;
    ea.c_out = s.c_mix;
    ea.ld_out = D;
    ea.wts = s.wts;
    if ((rc = launch_local_ent(ea, st))) return rc;
    if (tapping && (rc = tap_copy(tp.te, s.e_tanh, M * D * es, st))) return rc;
    if (tapping && (rc = tap_copy(tp.c, s.c_mix, M * D * es, st))) return rc;
    if ((rc = quant_te_c(s.e_tanh, s.c_mix, dt, M, D, p.bit_eps, s.xe, s.xc, st))) return rc;
  }
  if (tapping) {
    if ((rc = tap_codes(tp.q_te, tp.s_te, s.xe, M, st))) return rc;
    if ((rc = tap_codes(tp.q_c, tp.s_c, s.xc, M, st))) return rc;
  }
  // 5. decode caches (tesm.py:1235-1253)
  if (p.k_cache || p.v_cache) {
    CacheFillArgs cf;
    cf.dt = dt;
    cf.cdt = p.cache_dt;
    cf.B = p.B;
    cf.L = p.L;
    cf.R = R;
    cf.D = D;
    cf.W = p.cache_window > 0 ? p.cache_window : p.window;  // the ring's size (tesm.py:1243)
    cf.k = proj + o_k * es;
    cf.ld_k = n_in;
    cf.rope = static_cast<const float2*>(p.rope);
    cf.states = p.states;
    cf.ld_states = D;
    cf.k_cache = p.k_cache;
    cf.v_cache = p.v_cache;
    if ((rc = launch_cache_fill(cf, st))) return rc;
  }
  // 6. output gate and out_proj
  OutputPath op;
  op.xe = s.xe;
  op.xc = s.xc;
  op.xy = s.xy;
  op.yg = s.rowq ? nullptr : s.yg;
  op.state_proj = &p.state_proj;
  op.ent_proj = &p.ent_proj;
  op.out_proj = &p.out_proj;
  op.M = M;
  op.dm = dm;
  op.D = D;
  op.dt = dt;
  op.eps = p.bit_eps;
  op.local = proj + o_local * es;
  op.gate = proj + o_gate * es;
  op.ld = n_in;
  op.y = p.y;
  op.taps = tapping ? &tp : nullptr;
  return run_output_path(op, st);
}

// The dtype and size checks of a decode descriptor, made before any size is derived from it.
static int validate_siso_step_sizes(const tesm_hip_siso_step& p) {
  TESM_REQUIRE(p.dt == kF32 || p.dt == kBF16, kErrInvalidArg, "siso decode: dtype must be 0 or 1");
  // bounds that keep every size product of the step plan far inside int64
  TESM_REQUIRE(p.B <= (int64_t(1) << 31) && p.d_model <= (int64_t(1) << 20) && p.d_state <= (int64_t(1) << 20) &&
                   p.ent_rank <= (int64_t(1) << 20),
               kErrInvalidArg, "siso decode: sizes out of range");
  TESM_REQUIRE(p.B >= 1 && p.d_model >= 1 && p.d_state >= 1 && p.ent_rank >= 2 && p.ent_rank % 2 == 0 &&
                   p.window >= 1 && p.window <= 64 &&
                   (p.step_pos ? p.rope_rows >= 1 : p.seq_pos >= 0 && p.cache_idx >= 0 && p.cache_idx < p.window),
               kErrInvalidArg,
               "siso decode: bad sizes or ring position (need even ent_rank, 1 <= window <= 64, rope_rows >= 1 with "
               "step_pos)");
  return kOk;
}

int64_t tesm_hip_siso_decode_ws_bytes(const tesm_hip_siso_step* p) {
  if (!p || validate_siso_step_sizes(*p) != kOk) return -1;
  return plan_decode(*p, nullptr).total;
}

// Every check of a decode descriptor (shared by the entry points that run a step).
static int validate_siso_step(const tesm_hip_siso_step& p) {
  if (int rc = check_desc_ptrs(p)) return rc;
  if (int rc = validate_siso_step_sizes(p)) return rc;
  TESM_REQUIRE(p.u && p.decay_bias && p.local_bias && p.rope && p.state && p.state_out && p.k_cache && p.v_cache &&
                   p.y,
               kErrInvalidArg, "siso decode: null pointer");
  if (int rc = check_linear(p.in_proj, p.d_model, "in_proj")) return rc;
  if (int rc = check_linear(p.state_proj, p.d_state, "state_proj")) return rc;
  if (int rc = check_linear(p.ent_proj, p.d_state, "ent_proj")) return rc;
  if (int rc = check_linear(p.out_proj, p.d_model, "out_proj")) return rc;
  if (p.cross_state)
    if (int rc = check_linear(p.cross_q_proj, p.d_state, "cross_q_proj")) return rc;
  return kOk;
}

int tesm_hip_siso_decode(const tesm_hip_siso_step* pp, void* ws, int64_t ws_bytes, void* stream) {
  TESM_REQUIRE(pp != nullptr, kErrInvalidArg, "siso decode: null descriptor");
  if (int rc = validate_siso_step(*pp)) return rc;
  const tesm_hip_siso_step& p = *pp;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const DecodePlan s = plan_decode(p, ws);
  TESM_REQUIRE(ws && ws_bytes >= s.total, kErrWorkspace, "siso decode: workspace too small");
  tesm_hip_taps tp;
  const bool tapping = snapshot_taps(&tp);

  const int dt = p.dt;
  const int es = esize(dt);
  const int64_t Bn = p.B, dm = p.d_model, D = p.d_state, R = p.ent_rank;
  const int64_t n_in = 2 * dm + 3 * D + 2 * R;
  char* proj = static_cast<char*>(s.proj);
  const int64_t o_local = 0, o_sv = dm, o_decay = dm + D, o_write = dm + 2 * D, o_gate = dm + 3 * D,
                o_q = 2 * dm + 3 * D, o_k = 2 * dm + 3 * D + R;
  int rc;
  // 1. in_proj on the B new tokens
  const int64_t ld_u = p.ld_u > 0 ? p.ld_u : dm;
  TESM_REQUIRE(ld_u >= dm, kErrInvalidArg, "decode step: ld_u must be >= d_model");
  {
    LinearArgs la;
    la.op[0] = operand(s.xu, p.in_proj);
    la.M = Bn;
    la.N = n_in;
    la.Kp = kpad(dm);
    la.out = proj;
    la.out_dt = dt;
    la.ldo = n_in;
    if (!tapping && linear_fq_ok(la)) {  // quantization of u inside the product: one launch fewer per step
      FusedQuantIn f;
      f.x = p.u;
      f.ldx = ld_u;
      f.K = dm;
      f.eps = p.bit_eps;
      f.dt = dt;
      if ((rc = launch_linear_fq(la, f, st))) return rc;
    } else {
      if ((rc = launch_quant_act(p.u, dt, Bn, dm, ld_u, p.bit_eps, 1, s.xu.q, s.xu.ldq, s.xu.s, s.xu.rs, st)))
        return rc;
      if (tapping && (rc = tap_codes(tp.q_u, tp.s_u, s.xu, Bn, st))) return rc;
      if ((rc = launch_linear(la, st))) return rc;
    }
  }
  // 2. cross-layer query (tesm.py:1302-1305)
  if (p.cross_state) {
    if ((rc = launch_quant_act(p.cross_state, dt, Bn, D, D, p.bit_eps, 1, s.xs.q, s.xs.ldq, s.xs.s, s.xs.rs, st)))
      return rc;
    if (tapping && (rc = tap_codes(tp.q_cs, tp.s_cs, s.xs, Bn, st))) return rc;
    if ((rc = run_linear(s.xs, p.cross_q_proj, Bn, R, D, s.cq, dt, R, st))) return rc;
  }
  // 3. state update, ring write, window entanglement, codes of tanh(E) and C
  DecodeArgs da;
  da.dt = dt;
  da.cdt = p.cache_dt;
  da.B = Bn;
  da.R = R;
  da.D = D;
  da.W = p.window;
  if (p.step_pos) {  // read on the device at run time; the host fields only have to pass the checks
    da.step_pos = p.step_pos;
    da.rope_rows = p.rope_rows;
    da.pos = 0;
    da.slot = 0;
    da.valid = 1;
    da.full = 0;
  } else {
    da.pos = p.seq_pos;
    da.slot = p.cache_idx;
    da.valid = std::min<int64_t>(p.seq_pos + 1, p.window);
    da.full = da.valid >= p.window;
  }
  da.proj = proj;
  da.ld_proj = n_in;
  da.o_sv = o_sv;
  da.o_decay = o_decay;
  da.o_write = o_write;
  da.o_q = o_q;
  da.o_k = o_k;
  da.rope = static_cast<const float2*>(p.rope);
  da.decay_bias = p.decay_bias;
  da.bias = p.local_bias;
  da.q_add = s.cq;
  da.ld_qadd = R;
  da.thr = p.thr;
  da.ent_scale = p.ent_scale;
  da.eps = p.bit_eps;
  da.state = p.state;
  da.state_out = p.state_out;
  da.k_cache = p.k_cache;
  da.v_cache = p.v_cache;
  da.new_state = p.new_state;
  da.q_te = s.xe.q;
  da.s_te = s.xe.s;
  da.rs_te = s.xe.rs;
  da.q_c = s.xc.q;
  da.s_c = s.xc.s;
  da.rs_c = s.xc.rs;
  da.ldq = s.xe.ldq;
  if (tapping) da.tern = tp.tern;
  const bool tap_floats = tapping && tp.te && tp.c;
  if (tap_floats) {  // tanh(E) and C in dt to the taps, then quantized by their own kernels (same codes)
    da.q_te = nullptr;
    da.te_out = tp.te;
    da.c_out = tp.c;
    da.ld_out = D;
  }
  if ((rc = launch_decode_ent(da, st))) return rc;
  if (tap_floats) {
    if ((rc = launch_quant_act(tp.te, dt, Bn, D, D, p.bit_eps, 1, s.xe.q, s.xe.ldq, s.xe.s, s.xe.rs, st))) return rc;
    if ((rc = launch_quant_act(tp.c, dt, Bn, D, D, p.bit_eps, 1, s.xc.q, s.xc.ldq, s.xc.s, s.xc.rs, st))) return rc;
  }
  if (tapping) {
    if ((rc = tap_codes(tp.q_te, tp.s_te, s.xe, Bn, st))) return rc;
    if ((rc = tap_codes(tp.q_c, tp.s_c, s.xc, Bn, st))) return rc;
  }
  // 4. output gate and out_proj
  OutputPath op;
  op.xe = s.xe;
  op.xc = s.xc;
  op.xy = s.xy;
  op.yg = s.yg;
  op.state_proj = &p.state_proj;
  op.ent_proj = &p.ent_proj;
  op.out_proj = &p.out_proj;
  op.M = Bn;
  op.dm = dm;
  op.D = D;
  op.dt = dt;
  op.eps = p.bit_eps;
  op.local = proj + o_local * es;
  op.gate = proj + o_gate * es;
  op.ld = n_in;
  op.y = p.y;
  op.taps = tapping ? &tp : nullptr;
  if ((rc = run_output_path(op, st))) return rc;
  return p.step_pos ? launch_decode_advance(p.step_pos, p.window, st) : kOk;
}

int tesm_hip_siso_decode_noalloc(const tesm_hip_siso_step* p, void* stream) {
  TESM_REQUIRE(p != nullptr, kErrInvalidArg, "no-alloc decode: null descriptor");
  // the dtype and size errors of tesm_hip_siso_decode come before the scratch need is computed
  if (int rc = validate_siso_step_sizes(*p)) return rc;
  const int64_t need = plan_decode(*p, nullptr).total;
  TESM_REQUIRE(need <= kNoAllocScratchBytes, kErrWorkspace,
               "no-alloc decode: the step needs " + std::to_string(need) + " bytes of scratch, more than the " +
                   std::to_string(kNoAllocScratchBytes) + " of TESM_HIP_NOALLOC_SCRATCH_BYTES (use "
                   "tesm_hip_siso_decode with a workspace)");
  void* ptr = scratch_ptr();
  if (ptr == nullptr) return kErrLaunch;
  // every scratch byte the step reads is written earlier in the same step: nothing to clear
  return tesm_hip_siso_decode(p, ptr, kNoAllocScratchBytes, stream);
}

// Workspace layout of the MIMO decode step; with base == nullptr it only measures.
struct MimoDecodePlan {
  CodeBuf xu, xs, xe, xc, xy;
  void* proj;
  void* cq;
  void* te;  // (B, H*D) tanh(E) in dt
  void* cc;  // (B, H*D) C = E - S in dt
  void* yg;
  int64_t total;
};

MimoDecodePlan plan_mimo_decode(const tesm_hip_mimo_step& p, void* base) {
  Carve c(base);
  MimoDecodePlan s;
  const int64_t HD = p.n_heads * p.d_state;
  const int64_t n_in = 2 * p.d_model + 3 * HD + 2 * p.n_heads * p.ent_rank;
  const int es = esize(p.dt);
  s.xu = take_codes(c, p.B, p.d_model);
  s.proj = c.take<void>(p.B * n_in * es);
  if (p.cross_state) {
    s.xs = take_codes(c, p.B * p.n_heads, p.d_state);
    s.cq = c.take<void>(p.B * p.n_heads * p.ent_rank * es);
  } else {
    s.xs = CodeBuf{nullptr, nullptr, nullptr, 0};
    s.cq = nullptr;
  }
  s.te = c.take<void>(p.B * HD * es);
  s.cc = c.take<void>(p.B * HD * es);
  s.xe = take_codes(c, p.B, HD);
  s.xc = take_codes(c, p.B, HD);
  s.yg = p.d_model <= 1024 && p.B >= 256 ? nullptr : c.take<void>(p.B * p.d_model * es);
  s.xy = take_codes(c, p.B, p.d_model);
  s.total = c.off;
  return s;
}

int64_t tesm_hip_mimo_decode_ws_bytes(const tesm_hip_mimo_step* p) {
  if (!p) return -1;
  return plan_mimo_decode(*p, nullptr).total;
}

int tesm_hip_mimo_decode(const tesm_hip_mimo_step* pp, void* ws, int64_t ws_bytes, void* stream) {
  TESM_REQUIRE(pp != nullptr, kErrInvalidArg, "mimo decode: null descriptor");
  if (int rc = check_desc_ptrs(*pp)) return rc;
  const tesm_hip_mimo_step& p = *pp;
  hipStream_t st = static_cast<hipStream_t>(stream);
  TESM_REQUIRE(p.dt == kF32 || p.dt == kBF16, kErrInvalidArg, "mimo decode: dtype must be 0 or 1");
  TESM_REQUIRE(p.B >= 1 && p.d_model >= 1 && p.d_state >= 1 && p.n_heads >= 1 && p.ent_rank >= 2 &&
                   p.ent_rank % 2 == 0 && p.window >= 1 && p.window <= 64 && p.seq_pos >= 0 && p.cache_idx >= 0 &&
                   p.cache_idx < p.window,
               kErrInvalidArg,
               "mimo decode: bad sizes or ring position (need even ent_rank, 1 <= window <= 64)");
  TESM_REQUIRE(p.u && p.decay_bias && p.local_bias && p.rope && p.state && p.state_out && p.k_cache && p.v_cache &&
                   p.y,
               kErrInvalidArg, "mimo decode: null pointer");
  const int64_t Bn = p.B, dm = p.d_model, D = p.d_state, H = p.n_heads, R = p.ent_rank;
  const int64_t HD = H * D, HR = H * R;
  if (int rc = check_linear(p.in_proj, dm, "in_proj")) return rc;
  if (int rc = check_linear(p.state_proj, HD, "state_proj")) return rc;
  if (int rc = check_linear(p.ent_proj, HD, "ent_proj")) return rc;
  if (int rc = check_linear(p.out_proj, dm, "out_proj")) return rc;
  if (p.cross_state)
    if (int rc = check_linear(p.cross_q_proj, D, "cross_q_proj")) return rc;
  const MimoDecodePlan s = plan_mimo_decode(p, ws);
  TESM_REQUIRE(ws && ws_bytes >= s.total, kErrWorkspace, "mimo decode: workspace too small");
  tesm_hip_taps tp;
  const bool tapping = snapshot_taps(&tp);

  const int dt = p.dt;
  const int es = esize(dt);
  const int64_t n_in = 2 * dm + 3 * HD + 2 * HR;
  char* proj = static_cast<char*>(s.proj);
  const int64_t o_local = 0, o_sv = dm, o_decay = dm + HD, o_write = dm + 2 * HD, o_gate = dm + 3 * HD,
                o_q = 2 * dm + 3 * HD, o_k = 2 * dm + 3 * HD + HR;
  int rc;
  // 1. in_proj on the B new tokens (tesm_mimo.py:765-781)
  const int64_t ld_u = p.ld_u > 0 ? p.ld_u : dm;
  TESM_REQUIRE(ld_u >= dm, kErrInvalidArg, "mimo decode: ld_u must be >= d_model");
  {
    LinearArgs la;
    la.op[0] = operand(s.xu, p.in_proj);
    la.M = Bn;
    la.N = n_in;
    la.Kp = kpad(dm);
    la.out = proj;
    la.out_dt = dt;
    la.ldo = n_in;
    if (!tapping && linear_fq_ok(la)) {  // quantization of u inside the product: one launch fewer per step
      FusedQuantIn f;
      f.x = p.u;
      f.ldx = ld_u;
      f.K = dm;
      f.eps = p.bit_eps;
      f.dt = dt;
      if ((rc = launch_linear_fq(la, f, st))) return rc;
    } else {
      if ((rc = launch_quant_act(p.u, dt, Bn, dm, ld_u, p.bit_eps, 1, s.xu.q, s.xu.ldq, s.xu.s, s.xu.rs, st)))
        return rc;
      if (tapping && (rc = tap_codes(tp.q_u, tp.s_u, s.xu, Bn, st))) return rc;
      if ((rc = launch_linear(la, st))) return rc;
    }
  }
  // 2. cross-layer query per head: cross_q_proj over the B * n_heads state rows (tesm_mimo.py:818-826)
  if (p.cross_state) {
    if ((rc = launch_quant_act(p.cross_state, dt, Bn * H, D, D, p.bit_eps, 1, s.xs.q, s.xs.ldq, s.xs.s, s.xs.rs,
                               st)))
      return rc;
    if (tapping && (rc = tap_codes(tp.q_cs, tp.s_cs, s.xs, Bn * H, st))) return rc;
    if ((rc = run_linear(s.xs, p.cross_q_proj, Bn * H, R, D, s.cq, dt, R, st))) return rc;
  }
  // 3. per-head state update, ring write, window entanglement (tesm_mimo.py:838-887)
  DecodeArgs da;
  da.dt = dt;
  da.cdt = p.cache_dt;
  da.B = Bn;
  da.H = H;
  da.R = R;
  da.D = D;
  da.W = p.window;
  da.pos = p.seq_pos;
  da.slot = p.cache_idx;
  da.valid = std::min<int64_t>(p.seq_pos + 1, p.window);
  da.full = da.valid >= p.window;
  da.proj = proj;
  da.ld_proj = n_in;
  da.o_sv = o_sv;
  da.o_decay = o_decay;
  da.o_write = o_write;
  da.o_q = o_q;
  da.o_k = o_k;
  da.rope = static_cast<const float2*>(p.rope);
  da.decay_bias = p.decay_bias;
  da.bias = p.local_bias;
  da.q_add = s.cq;
  da.ld_qadd = R;
  da.thr = p.thr;
  da.ent_scale = p.ent_scale;
  da.eps = p.bit_eps;
  da.state = p.state;
  da.state_out = p.state_out;
  da.k_cache = p.k_cache;
  da.v_cache = p.v_cache;
  da.new_state = p.new_state;
  da.te_out = s.te;
  da.c_out = s.cc;
  da.ld_out = HD;
  if (tapping) da.tern = tp.tern;
  if ((rc = launch_decode_ent(da, st))) return rc;
  // 4. per-token codes of tanh(E) and C over the flattened heads (tesm_mimo.py:895-900)
  if ((rc = quant_te_c(s.te, s.cc, dt, Bn, HD, p.bit_eps, s.xe, s.xc, st))) return rc;
  if (tapping) {
    if ((rc = tap_copy(tp.te, s.te, Bn * HD * es, st))) return rc;
    if ((rc = tap_copy(tp.c, s.cc, Bn * HD * es, st))) return rc;
    if ((rc = tap_codes(tp.q_te, tp.s_te, s.xe, Bn, st))) return rc;
    if ((rc = tap_codes(tp.q_c, tp.s_c, s.xc, Bn, st))) return rc;
  }
  // 5. output gate and out_proj (tesm_mimo.py:902-906)
  OutputPath op;
  op.xe = s.xe;
  op.xc = s.xc;
  op.xy = s.xy;
  op.yg = s.yg;
  op.state_proj = &p.state_proj;
  op.ent_proj = &p.ent_proj;
  op.out_proj = &p.out_proj;
  op.M = Bn;
  op.dm = dm;
  op.D = HD;
  op.dt = dt;
  op.eps = p.bit_eps;
  op.local = proj + o_local * es;
  op.gate = proj + o_gate * es;
  op.ld = n_in;
  op.y = p.y;
  op.taps = tapping ? &tp : nullptr;
  return run_output_path(op, st);
}

int tesm_hip_mimo_coef(const void* mimo_x, const void* mimo_o, int dt, int64_t n_heads, int64_t mimo_rank,
                       int64_t d_state, float* coef, float* x0sq, void* stream) {
  if (int rc = check_ptrs("mimo_coef", {{mimo_x, "mimo_x"}, {mimo_o, "mimo_o"}, {coef, "coef"}, {x0sq, "x0sq"}})) return rc;
  return launch_mimo_coef(mimo_x, mimo_o, dt, n_heads, mimo_rank, d_state, coef, x0sq,
                          static_cast<hipStream_t>(stream));
}

int64_t tesm_hip_mimo_prefill_ws_bytes(const tesm_hip_mimo_layer* p) {
  if (!p) return -1;
  return plan_mimo(*p, nullptr).total;
}

int tesm_hip_mimo_prefill(const tesm_hip_mimo_layer* pp, void* ws, int64_t ws_bytes, void* stream) {
  TESM_REQUIRE(pp != nullptr, kErrInvalidArg, "mimo layer: null descriptor");
  if (int rc = check_desc_ptrs(*pp)) return rc;
  const tesm_hip_mimo_layer& p = *pp;
  hipStream_t st = static_cast<hipStream_t>(stream);
  TESM_REQUIRE(p.dt == kF32 || p.dt == kBF16, kErrInvalidArg, "mimo layer: dtype must be 0 or 1");
  TESM_REQUIRE(p.B >= 1 && p.L >= 1 && p.d_model >= 1 && p.d_state >= 1 && p.n_heads >= 1 && p.ent_rank >= 2 &&
                   p.ent_rank % 2 == 0 && p.window >= 0 && p.window <= 64,
               kErrInvalidArg, "mimo layer: bad sizes (need even ent_rank, 0 <= window <= 64)");
  TESM_REQUIRE(p.u && p.decay_bias && (p.local_bias || p.window == 0) && p.rope && p.mimo_coef && p.mimo_x0sq && p.y,
               kErrInvalidArg, "mimo layer: null pointer");
  TESM_REQUIRE(p.window > 0 || (p.global_embed && p.global_dim >= 1 && p.global_scale && p.global_bias),
               kErrInvalidArg, "mimo layer: global entanglement (window 0) needs the relative-position parameters");
  TESM_REQUIRE(p.cache_window >= 0 && (p.window > 0 || p.cache_window > 0 || !(p.k_cache || p.v_cache)),
               kErrInvalidArg, "mimo layer: a cache with window 0 needs cache_window");
  const int64_t H = p.n_heads, D = p.d_state, R = p.ent_rank, dm = p.d_model, HD = H * D, HR = H * R;
  if (int rc = check_linear(p.in_proj, dm, "in_proj")) return rc;
  if (int rc = check_linear(p.state_proj, HD, "state_proj")) return rc;
  if (int rc = check_linear(p.ent_proj, HD, "ent_proj")) return rc;
  if (int rc = check_linear(p.out_proj, dm, "out_proj")) return rc;
  const MimoPlan s = plan_mimo(p, ws);
  TESM_REQUIRE(ws && ws_bytes >= s.total, kErrWorkspace, "mimo layer: workspace too small");
  tesm_hip_taps tp;
  const bool tapping = snapshot_taps(&tp);

  const int dt = p.dt;
  const int es = esize(dt);
  const int64_t M = p.B * p.L;
  const int64_t n_in = 2 * dm + 3 * HD + 2 * HR;
  char* proj = static_cast<char*>(s.proj);
  // slice offsets of the in_proj output (tesm_mimo.py:940-949)
  const int64_t o_local = 0, o_sv = dm, o_decay = dm + HD, o_write = dm + 2 * HD, o_gate = dm + 3 * HD,
                o_q = 2 * dm + 3 * HD, o_k = 2 * dm + 3 * HD + HR;
  int rc;
  // 1. in_proj
  // the u quantization also clears the single-pass scan's flags, saving the scan its reset launch
  int* scan_zero = nullptr;
  int64_t scan_zero_n = 0;
  scan_lb_clear_range(p.B, p.L, HD, kMimoScanChunk, s.scan_ws, &scan_zero, &scan_zero_n);
  if ((rc = launch_quant_act(p.u, dt, M, dm, dm, p.bit_eps, 1, s.xu.q, s.xu.ldq, s.xu.s, s.xu.rs, st, scan_zero,
                             scan_zero_n)))
    return rc;
  if (tapping && (rc = tap_codes(tp.q_u, tp.s_u, s.xu, M, st))) return rc;
  // in_proj with the scan's gates applied in its epilogue (tesm_mimo.py:958-961) where its kernels
  // allow it (M > 32 and 32-column aligned regions), so the scan only streams them; else the scan
  // applies them to the raw slices.  TESM_HIP_NO_GATE_EPI=1 keeps the latter (a diagnostic switch,
  // read per call, for side-by-side timing and bit-for-bit comparison: the values are the same).
  const char* no_gate_epi = std::getenv("TESM_HIP_NO_GATE_EPI");
  const bool gate_epi = M > 32 && dm % 32 == 0 && HD % 32 == 0 && !(no_gate_epi && no_gate_epi[0] == '1');
  {
    LinearArgs la;
    la.op[0] = operand(s.xu, p.in_proj);
    la.M = M;
    la.N = n_in;
    la.Kp = kpad(dm);
    la.out = proj;
    la.out_dt = dt;
    la.ldo = n_in;
    if (gate_epi) {
      la.epilogue = kEpiGates;
      la.act_n0 = o_sv;  // state value, then decay, then write (o_decay = o_sv + HD, o_write = o_sv + 2 HD)
      la.act_w = HD;
      la.act_bias = p.decay_bias;
    }
    if ((rc = launch_linear(la, st))) return rc;
  }
  // 2. rank-free state scan: sequential float32 recurrence h = d h + w tanh(sv) per channel
  ScanArgs sa;
  sa.mode = gate_epi ? 2 : 1;
  sa.dt = dt;
  sa.out_dt = kF32;
  sa.clamp = 0;
  sa.round_update = 0;
  sa.B = p.B;
  sa.L = p.L;
  sa.C = HD;
  sa.cs = kMimoScanChunk;
  sa.decay = proj + o_decay * es;
  sa.ld_decay = n_in;
  sa.update = proj + o_write * es;
  sa.ld_update = n_in;
  sa.sv = proj + o_sv * es;
  sa.ld_sv = n_in;
  sa.decay_bias = p.decay_bias;
  sa.states = s.S;
  sa.ld_states = HD;
  sa.flags_clear = scan_zero_n > 0;
  if ((rc = launch_scan(sa, s.scan_ws, s.scan_bytes, st))) return rc;
  if ((rc = launch_mimo_final(s.S, p.mimo_x0sq, p.B, p.L, HD, p.h_final, p.last_state, st))) return rc;
  if (tapping && (rc = tap_copy(tp.S, s.S, M * HD * 4, st))) return rc;
  const void* q_raw = proj + o_q * es;
  const void* k_raw = proj + o_k * es;
  if (p.window > 0) {
    // 3. per-head window scores, strict ternary, count normalisation (tesm_mimo.py:536-586)
    EntArgs ea;
    ea.dt = dt;
    ea.mimo = 1;
    ea.B = p.B;
    ea.L = p.L;
    ea.H = H;
    ea.R = R;
    ea.D = D;
    ea.W = p.window;
    ea.q = q_raw;
    ea.ld_q = n_in;
    ea.k = k_raw;
    ea.ld_k = n_in;
    ea.rope = static_cast<const float2*>(p.rope);
    ea.bias = p.local_bias;
    ea.thr = p.thr;
    ea.ent_scale = p.ent_scale;
    ea.S = s.S;
    ea.ld_s = HD;
    ea.wts = s.wts;
    if (tapping) ea.tern = tp.tern;
    if ((rc = launch_local_ent(ea, st))) return rc;
    // 4. window mix, entangled state, rank merge; tanh(E c) and C c in dt for the projections
    MimoMixArgs ma;
    ma.dt = dt;
    ma.B = p.B;
    ma.L = p.L;
    ma.H = H;
    ma.D = D;
    ma.W = p.window;
    ma.S = s.S;
    ma.wts = s.wts;
    ma.coef = p.mimo_coef;
    ma.ent_scale = p.ent_scale;
    ma.te = s.te;
    ma.cc = s.cc;
    if ((rc = launch_mimo_mix(ma, st))) return rc;
    if (tapping && (rc = tap_copy(tp.wts, s.wts, M * H * p.window * 4, st))) return rc;
  } else {
    // 3-4. global causal entanglement over the flattened heads (tesm_mimo.py:655-687), E = A, merged
    if ((rc = launch_global_bias_table(dt, 2 * p.L, p.global_embed, p.global_dim, p.global_scale, p.global_bias,
                                       s.g_table, st)))
      return rc;
    GlobalArgs ga;
    ga.dt = dt;
    ga.mimo = 1;
    ga.B = p.B;
    ga.L = p.L;
    ga.H = H;
    ga.R = R;
    ga.D = D;
    ga.q = q_raw;
    ga.ld_q = n_in;
    ga.k = k_raw;
    ga.ld_k = n_in;
    ga.rope = static_cast<const float2*>(p.rope);
    ga.table = s.g_table;
    ga.thr = p.thr;
    ga.sqrt_div = static_cast<float>(std::sqrt(static_cast<double>(HR)));
    ga.S = s.S;
    ga.ld_s = HD;
    ga.coef = p.mimo_coef;
    ga.e_tanh = s.te;
    ga.c_out = s.cc;
    ga.ld_out = HD;
    ga.tern = s.g_tern;
    ga.count = s.g_count;
    ga.qr = s.g_qr;
    ga.kr = s.g_kr;
    if ((rc = launch_global_ent(ga, st))) return rc;
    if (tapping && (rc = tap_copy(tp.tern, s.g_tern, M * global_tern_pitch(p.L), st))) return rc;
  }
  if (p.stats_ternary || p.stats_counts) {  // tesm_mimo.py:1019-1020 -> 458-523
    MimoStatsArgs sa2;
    sa2.dt = dt;
    sa2.global = p.window == 0;
    sa2.B = p.B;
    sa2.L = p.L;
    sa2.H = H;
    sa2.R = R;
    sa2.W = p.window > 0 ? std::min<int64_t>(p.window, p.L) : 0;
    sa2.S = std::min<int64_t>(p.L, p.window > 0 ? 64 : 32);
    sa2.q = q_raw;
    sa2.ld_q = n_in;
    sa2.k = k_raw;
    sa2.ld_k = n_in;
    sa2.rope = static_cast<const float2*>(p.rope);
    sa2.sqrt_r = static_cast<float>(std::sqrt(static_cast<double>(R)));
    sa2.thr = p.thr;
    sa2.ternary = p.stats_ternary;
    sa2.counts = p.stats_counts;
    if ((rc = launch_mimo_stats(sa2, st))) return rc;
  }
  if ((rc = quant_te_c(s.te, s.cc, dt, M, HD, p.bit_eps, s.xe, s.xc, st))) return rc;
  if (tapping) {
    if ((rc = tap_copy(tp.te, s.te, M * HD * es, st))) return rc;
    if ((rc = tap_copy(tp.c, s.cc, M * HD * es, st))) return rc;
    if ((rc = tap_codes(tp.q_te, tp.s_te, s.xe, M, st))) return rc;
    if ((rc = tap_codes(tp.q_c, tp.s_c, s.xc, M, st))) return rc;
  }
  // 5. decode caches
  if (p.k_cache || p.v_cache) {
    CacheFillArgs cf;
    cf.dt = dt;
    cf.cdt = p.cache_dt;
    cf.sdt = kF32;
    cf.B = p.B;
    cf.L = p.L;
    cf.H = H;
    cf.R = R;
    cf.D = D;
    cf.W = p.cache_window > 0 ? p.cache_window : p.window;  // the ring's size (tesm_mimo.py:1028)
    cf.k = proj + o_k * es;
    cf.ld_k = n_in;
    cf.rope = static_cast<const float2*>(p.rope);
    cf.states = s.S;
    cf.ld_states = HD;
    cf.vscale = p.mimo_x0sq;
    cf.k_cache = p.k_cache;
    cf.v_cache = p.v_cache;
    if ((rc = launch_cache_fill(cf, st))) return rc;
  }
  // 6. output gate and out_proj
  OutputPath op;
  op.xe = s.xe;
  op.xc = s.xc;
  op.xy = s.xy;
  op.yg = s.yg;
  op.state_proj = &p.state_proj;
  op.ent_proj = &p.ent_proj;
  op.out_proj = &p.out_proj;
  op.M = M;
  op.dm = dm;
  op.D = HD;
  op.dt = dt;
  op.eps = p.bit_eps;
  op.local = proj + o_local * es;
  op.gate = proj + o_gate * es;
  op.ld = n_in;
  op.y = p.y;
  op.taps = tapping ? &tp : nullptr;
  return run_output_path(op, st);
}

// ---------------------------------------------------------------------------
// RMSNorm and FeedForward of the TESM block
// ---------------------------------------------------------------------------
int tesm_hip_add_rmsnorm(const tesm_hip_rmsnorm* pp, void* stream) {
  TESM_REQUIRE(pp != nullptr, kErrInvalidArg, "rmsnorm: null descriptor");
  if (int rc = check_desc_ptrs(*pp)) return rc;
  const tesm_hip_rmsnorm& p = *pp;
  NormArgs a;
  a.dt = p.dt;
  a.M = p.M;
  a.D = p.D;
  a.eps = p.eps;
  a.x = p.x;
  a.ld_x = p.ld_x > 0 ? p.ld_x : p.D;
  a.res = p.residual;
  a.res_dt = p.residual_dt;
  a.ld_res = p.ld_res > 0 ? p.ld_res : p.D;
  a.res_out = p.residual_out;
  a.res_out_dt = p.residual_out_dt;
  a.ld_res_out = p.ld_res_out > 0 ? p.ld_res_out : p.D;
  a.weight = p.weight;
  a.y = p.y;
  a.ld_y = p.ld_y > 0 ? p.ld_y : p.D;
  a.q = p.q;
  a.ldq = p.ldq;
  a.s_x = p.s_x;
  a.rowsum = p.rowsum;
  a.bit_eps = p.bit_eps;
  return launch_add_rmsnorm(a, static_cast<hipStream_t>(stream));
}


int64_t tesm_hip_ffn_ws_bytes(const tesm_hip_ffn* p) {
  if (!p) return -1;
  return plan_ffn(*p, nullptr).total;
}

int tesm_hip_ffn_forward(const tesm_hip_ffn* pp, void* ws, int64_t ws_bytes, void* stream) {
  TESM_REQUIRE(pp != nullptr, kErrInvalidArg, "ffn: null descriptor");
  if (int rc = check_desc_ptrs(*pp)) return rc;
  const tesm_hip_ffn& p = *pp;
  hipStream_t st = static_cast<hipStream_t>(stream);
  TESM_REQUIRE(p.dt == kF32 || p.dt == kBF16, kErrInvalidArg, "ffn: dtype must be 0 or 1");
  TESM_REQUIRE(p.M >= 0 && p.d_model >= 1 && p.d_inter >= 1, kErrInvalidArg, "ffn: bad sizes");
  TESM_REQUIRE(p.y && p.ld_y >= p.d_model, kErrInvalidArg, "ffn: need y with ld_y >= d_model");
  if (p.x_codes)
    TESM_REQUIRE(p.x_scale && p.x_rowsum && p.ldq_x >= kpad(p.d_model) && p.ldq_x % 16 == 0, kErrInvalidArg,
                 "ffn: x codes need x_scale, x_rowsum and ldq_x >= kpad(d_model), a multiple of 16");
  else
    TESM_REQUIRE(p.x && p.ld_x >= p.d_model, kErrInvalidArg, "ffn: need x (ld_x >= d_model) or x codes");
  if (int rc = check_linear(p.gate_proj, p.d_model, "gate_proj")) return rc;
  if (int rc = check_linear(p.up_proj, p.d_model, "up_proj")) return rc;
  if (int rc = check_linear(p.down_proj, p.d_inter, "down_proj")) return rc;
  const FfnPlan s = plan_ffn(p, ws);
  TESM_REQUIRE(ws && ws_bytes >= s.total, kErrWorkspace, "ffn: workspace too small");
  if (p.M == 0) return kOk;
  tesm_hip_taps tp;
  const bool tapping = snapshot_taps(&tp);
  int rc;
  CodeBuf xq = s.xq;
  if (p.x_codes) {
    xq = CodeBuf{const_cast<int8_t*>(p.x_codes), const_cast<float*>(p.x_scale), const_cast<int32_t*>(p.x_rowsum),
                 p.ldq_x};
  } else if ((rc = launch_quant_act(p.x, p.dt, p.M, p.d_model, p.ld_x, p.bit_eps, 1, xq.q, xq.ldq, xq.s, xq.rs, st))) {
    return rc;
  }
  if (tapping && (rc = tap_codes(tp.q_u, tp.s_u, xq, p.M, st))) return rc;
  // gate and up products on the same codes, h = silu(gate) * up (mixer_seq_simple.py:57-64)
  LinearArgs g;
  g.op[0] = operand(xq, p.gate_proj);
  g.op[1] = operand(xq, p.up_proj);
  g.M = p.M;
  g.N = p.d_inter;
  g.Kp = kpad(p.d_model);
  g.out = s.h;
  g.ldo = p.d_inter;
  g.out_dt = p.dt;
  g.epilogue = kEpiSwiGLU;
  if ((rc = launch_linear(g, st))) return rc;
  // down_proj(h) (mixer_seq_simple.py:65)
  if ((rc = launch_quant_act(s.h, p.dt, p.M, p.d_inter, p.d_inter, p.bit_eps, 1, s.hq.q, s.hq.ldq, s.hq.s, s.hq.rs,
                             st)))
    return rc;
  if (tapping && (rc = tap_codes(tp.q_h, tp.s_h, s.hq, p.M, st))) return rc;
  return run_linear(s.hq, p.down_proj, p.M, p.d_model, p.d_inter, p.y, p.dt, p.ld_y, st);
}

}  // extern "C"
