// C ABI of libtjev_gdn.so (declared in include/tjev_gdn.h): argument validation with the
// reference's error conventions, the workspace layout, and dispatch to the compiled
// (chunk, head dim, precision, dtype) kernel sequences.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/tjev_gdn.h"
#include "gdn_launch.h"

namespace {

thread_local std::string g_error;

int fail(int status, const std::string& msg) {
  g_error = msg;
  return status;
}

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

const gdn::ShapeTable* lookup(int c, int d) {
#define GDN_SHAPE(cc, dd) \
  if (c == cc && d == dd) return gdn::table_##cc##_##dd();
#include "gdn_shapes.def"
#undef GDN_SHAPE
  return nullptr;
}

std::string supported_shapes() {
  std::string s;
#define GDN_SHAPE(cc, dd) s += "(chunk " #cc ", dim " #dd ") ";
#include "gdn_shapes.def"
#undef GDN_SHAPE
  return s;
}

// The chunk the kernels run: the requested one, 16 for chunks below 16 and 128 for chunks above
// 128 (the chunked form is exact for any chunk, so only fp32 rounding depends on it; a chunk's
// C x C operands in LDS bound it at 128).
int kernel_chunk(const tjev_gdn_params* p) { return p->chunk < 16 ? 16 : (p->chunk > 128 ? 128 : p->chunk); }

// Validation in the order of gdn_megakernel (pallas_tpu_mega.py:597-615) and
// heads_per_block (pallas_tpu_v2.py:518-525).
int validate(const tjev_gdn_params* p) {
  if (!p) return fail(TJEV_GDN_EINVAL, "null params");
  if (p->precision < 0 || p->precision > 3)
    return fail(TJEV_GDN_EINVAL, "precision in (highest, high, bf16, mixed)");
  if (p->inverse < 0 || p->inverse > 1)
    return fail(TJEV_GDN_EINVAL, "the GDN megakernel's inverse in (doubling, blocked)");
  if (!pow2(p->chunk) || p->chunk < 8)
    return fail(TJEV_GDN_EINVAL, "the GDN megakernel needs a power-of-two chunk >= 8, not " +
                                     std::to_string(p->chunk));
  if (p->batch <= 0 || p->length <= 0 || p->key_heads <= 0 || p->value_heads <= 0 ||
      p->key_dim <= 0 || p->value_dim <= 0)
    return fail(TJEV_GDN_EINVAL, "batch, length, heads and dims must be positive");
  if (p->value_heads % p->key_heads)
    return fail(TJEV_GDN_EINVAL, std::to_string(p->value_heads) + " value heads are not groups of " +
                                     std::to_string(p->key_heads) + " key heads");
  if (p->taps < 0 || p->taps > 5)
    return fail(TJEV_GDN_EINVAL, "conv kernel of " + std::to_string(p->taps) +
                                     " taps: the megakernel supports 1..5");
  if (p->io_dtype < 0 || p->io_dtype > 1 || p->gate_dtype < 0 || p->gate_dtype > 1)
    return fail(TJEV_GDN_EINVAL, "dtypes must be TJEV_GDN_F32 or TJEV_GDN_BF16");
  if (p->heads_per_step < 0) return fail(TJEV_GDN_EINVAL, "heads_per_step must be >= 0");
  if (p->qk_dtype < 0 || p->qk_dtype > 1) return fail(TJEV_GDN_EINVAL, "qk_dtype must be TJEV_GDN_F32 or TJEV_GDN_BF16");
  if (p->residuals < TJEV_GDN_SAVE_STATES || p->residuals > TJEV_GDN_SAVE_ALL)
    return fail(TJEV_GDN_EINVAL, "residuals must be TJEV_GDN_SAVE_STATES, _TINV or _ALL");
  if (p->key_dim != p->value_dim)
    return fail(TJEV_GDN_EUNSUPPORTED, "this build's kernels need key_dim == value_dim");
  if (!lookup(kernel_chunk(p), p->key_dim))
    return fail(TJEV_GDN_EUNSUPPORTED, "no kernels for chunk " + std::to_string(p->chunk) + ", head dim " +
                                           std::to_string(p->key_dim) + "; compiled: " + supported_shapes());
  const long w = 2L * p->key_heads * p->key_dim + (long)p->value_heads * p->value_dim;
  if (w > (1L << 30) || (long)p->batch * p->length * w > (1L << 40))
    return fail(TJEV_GDN_EINVAL, "problem too large");
  // the flat grids: k_prep / k_post launch B * N * (2 Hk + H) workgroups of 256 work-items and
  // k_bwd_grads B * H * N of 4 C; a launch holds fewer than 2^32 work-items along x
  const long C = kernel_chunk(p), n = (p->length + C - 1) / C;
  const long slots = 2L * p->key_heads + p->value_heads;
  if ((long)p->batch * n * slots * 256 >= (1L << 32) || (long)p->batch * p->value_heads * n * 4 * C >= (1L << 32))
    return fail(TJEV_GDN_EUNSUPPORTED, "batch * chunks * heads too large for one launch of this build's grids");
  return 0;
}

struct Layout {
  size_t segp, qn, kn, vv, gam, gaml, bet, uu, ww, vnew, s_last, tt, qk, xl, kt, gg, gsp, dqh, dkh, dgam, dkws, dcross,
      dbet, pa, pd, dwp;
  size_t total;
};

size_t up(size_t x) { return (x + 255) & ~size_t(255); }

// bytes per element of the chunk-boundary states: bf16 when the state-path products are one
// bf16 pass (mixed, bf16), as the reference keeps them (pallas_tpu_mega.py:425-426)
size_t state_elem(const tjev_gdn_params* p) {
  return (p->precision == TJEV_GDN_MIXED || p->precision == TJEV_GDN_ONE_PASS_BF16) ? 2 : 4;
}
// bytes per element of T: bf16 when the intra-chunk products are one bf16 pass (bf16)
size_t tinv_elem(const tjev_gdn_params* p) { return p->precision == TJEV_GDN_ONE_PASS_BF16 ? 2 : 4; }

// Whether the forward's kernels build v (k_chunk) and, with one value head per key head, q
// (k_out) from the raw rows: bf16 I/O, a conv of 1 to 4 taps and the 128-token kernels at head
// dim 128, the launch sequence's rule (gdn_inst.hip). Such a forward's workspace holds no fp32 v
// (q) rows. The LDS-poison debug library keeps them and builds them in k_chunk and k_out unless
// TJEV_GDN_UNFUSED=1 is set (read on each call): the route through k_prep's rows, the fused
// route's bitwise reference.
bool fwd_fuses_v(const tjev_gdn_params* p) {
  return p->io_dtype == TJEV_GDN_BF16 && kernel_chunk(p) == 128 && p->key_dim == 128 && p->value_dim == 128 &&
         p->taps >= 1 && p->taps <= 4;
}
bool fwd_fuses_q(const tjev_gdn_params* p) { return fwd_fuses_v(p) && p->value_heads == p->key_heads; }
#ifdef GDN_LDS_POISON
constexpr bool kKeepRows = true;
bool unfused() {
  const char* e = getenv("TJEV_GDN_UNFUSED");
  return e && e[0] == '1';
}
#else
constexpr bool kKeepRows = false;
#endif

Layout layout(const tjev_gdn_params* p, int backward) {
  const size_t C = kernel_chunk(p), D = p->key_dim;
  const size_t B = p->batch, H = p->value_heads, Hk = p->key_heads;
  const size_t N = (p->length + C - 1) / C, Tp = N * C;
  const size_t W = 2 * Hk * D + H * D;
  const size_t ntiles = D / (D < 32 ? D : 32);
  const size_t hv = B * H * Tp * D * 4, hkv = B * Hk * Tp * D * 4, tok = B * H * Tp * 4;
  Layout L{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += up(bytes);
    return at;
  };
  const size_t none = ~size_t(0);
  const bool drop_q = !backward && !kKeepRows && fwd_fuses_q(p), drop_v = !backward && !kKeepRows && fwd_fuses_v(p);
  L.segp = take(B * Tp * 4);
  L.qn = drop_q ? none : take(hkv);
  L.kn = take(hkv);
  L.vv = drop_v ? none : take(hv);
  L.gam = take(tok);
  L.gaml = take(tok);
  L.bet = take(tok);
  L.vnew = p->residuals == TJEV_GDN_SAVE_ALL ? none : take(hv);  // else a residual
  if (!backward) {
    L.uu = take(hv);
    L.ww = take(hv);
    // bf16 states: the fp32 state before each row's last chunk, for the final state
    L.s_last = state_elem(p) == 2 ? take(B * H * D * D * 4) : none;
    L.tt = L.qk = L.xl = L.kt = L.gg = L.gsp = L.dqh = L.dkh = L.dgam = L.dkws = L.dcross = L.dbet = L.pa = L.pd = L.dwp =
        none;
  } else {
    L.uu = L.ww = L.s_last = none;
    L.tt = p->residuals == TJEV_GDN_SAVE_STATES ? take(B * H * N * C * C * tinv_elem(p)) : none;
    L.qk = take(B * H * N * C * C * 4);
    L.xl = take(hv);
    L.kt = take(hv);
    L.gg = take(B * H * N * D * D * 4);
    L.gsp = take(B * H * N * ntiles * 4);
    L.dqh = take(hv);
    L.dkh = take(hv);
    L.dgam = take(tok);
    L.dkws = take(tok);
    L.dcross = take(tok);
    L.dbet = take(tok);
    L.pa = take(B * N * H * 8);
    L.pd = take(B * N * H * 8);
    L.dwp = take(B * N * (p->taps > 0 ? p->taps : 1) * W * 4);
  }
  L.total = o;
  return L;
}

// the residual buffer: states, then T and v_new as p->residuals keeps them
struct Residuals {
  size_t states, tinv, vnew, total;
};

Residuals residual_layout(const tjev_gdn_params* p) {
  const size_t C = kernel_chunk(p), D = p->key_dim;
  const size_t B = p->batch, H = p->value_heads;
  const size_t N = (p->length + C - 1) / C;
  const size_t none = ~size_t(0);
  Residuals R{};
  R.states = 0;
  size_t o = up(B * H * N * D * D * state_elem(p));
  R.tinv = R.vnew = none;
  if (p->residuals >= TJEV_GDN_SAVE_TINV) {
    R.tinv = o;
    o += up(B * H * N * C * C * tinv_elem(p));
  }
  if (p->residuals == TJEV_GDN_SAVE_ALL) {
    R.vnew = o;
    o += up(B * H * N * C * D * 4);
  }
  R.total = o;
  return R;
}

template <class T>
T* at(void* ws, size_t off) {
  return off == ~size_t(0) ? nullptr : reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

gdn::GdnArgs base_args(const tjev_gdn_params* p, void* ws, const Layout& L) {
  gdn::GdnArgs A{};
  const int C = kernel_chunk(p), D = p->key_dim;
  A.B = p->batch;
  A.T = p->length;
  A.N = (p->length + C - 1) / C;
  A.Tp = A.N * C;
  A.Hk = p->key_heads;
  A.H = p->value_heads;
  A.ratio = p->value_heads / p->key_heads;
  A.taps = p->taps;
  A.W = 2 * p->key_heads * D + p->value_heads * D;
  A.ntiles = D / (D < 32 ? D : 32);
  A.scale = 1.0f / sqrtf((float)D);
  A.segp = at<int32_t>(ws, L.segp);
  A.qn = at<float>(ws, L.qn);
  A.kn = at<float>(ws, L.kn);
  A.vv = at<float>(ws, L.vv);
  A.gam = at<float>(ws, L.gam);
  A.gaml = at<float>(ws, L.gaml);
  A.bet = at<float>(ws, L.bet);
  A.uu = at<float>(ws, L.uu);
  A.ww = at<float>(ws, L.ww);
  A.vnew = at<float>(ws, L.vnew);
  A.s_last = at<float>(ws, L.s_last);
  A.tt = at<float>(ws, L.tt);
  A.qk = at<float>(ws, L.qk);
  A.xl = at<float>(ws, L.xl);
  A.kt = at<float>(ws, L.kt);
  A.gg = at<float>(ws, L.gg);
  A.gsp = at<float>(ws, L.gsp);
  A.dqh = at<float>(ws, L.dqh);
  A.dkh = at<float>(ws, L.dkh);
  A.dgam = at<float>(ws, L.dgam);
  A.dkws = at<float>(ws, L.dkws);
  A.dcross = at<float>(ws, L.dcross);
  A.dbet = at<float>(ws, L.dbet);
  A.pa = at<double>(ws, L.pa);
  A.pd = at<double>(ws, L.pd);
  A.dwp = at<float>(ws, L.dwp);
  A.res = p->residuals;
  A.inv = p->inverse;
#ifdef GDN_LDS_POISON
  A.fuse_v = !unfused();
#else
  A.fuse_v = 1;
#endif
  return A;
}

// the residual parts into the arguments (T and v_new there instead of in the workspace)
void bind_residuals(const tjev_gdn_params* p, float* res, gdn::GdnArgs& A) {
  const Residuals R = residual_layout(p);
  A.states = res;
  if (R.tinv != ~size_t(0)) A.tt = at<float>(res, R.tinv);
  if (R.vnew != ~size_t(0)) A.vnew = at<float>(res, R.vnew);
}

int aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---- per-kernel timing: an event pair around each launch while profiling is on
const char* const kKernelNames[gdn::K_COUNT] = {
    "gdn_prep_fwd", "gdn_chunk_fwd", "gdn_scan_fwd", "gdn_out",       "gdn_prep_bwd",   "gdn_chunk_bwd",
    "gdn_bwd_local", "gdn_scan_bwd", "gdn_bwd_grads", "gdn_post",     "gdn_reduce",     "gdn_norm_fwd",
    "gdn_norm_bwd",  "gdn_norm_reduce", "gdn_final_state", "gdn_decode"};

struct Profiler {
  bool on = false;
  std::vector<std::pair<int, std::pair<hipEvent_t, hipEvent_t>>> marks;
  std::vector<hipEvent_t> pool;
  hipEvent_t pending = nullptr;
  hipError_t err = hipSuccess;
  hipEvent_t take() {
    if (!pool.empty()) {
      hipEvent_t e = pool.back();
      pool.pop_back();
      return e;
    }
    hipEvent_t e = nullptr;
    const hipError_t r = hipEventCreate(&e);
    if (r != hipSuccess) err = r;
    return e;
  }
};
Profiler g_prof;

void prof_mark(void*, int kernel, int end, hipStream_t st) {
  hipEvent_t e = g_prof.take();
  if (!e) return;
  const hipError_t r = hipEventRecord(e, st);
  if (r != hipSuccess) g_prof.err = r;
  if (!end) {
    g_prof.pending = e;
  } else {
    g_prof.marks.push_back({kernel, {g_prof.pending, e}});
    g_prof.pending = nullptr;
  }
}

const gdn::Timer g_timer{prof_mark, nullptr};

// ---- the poison debug mode: with TJEV_GDN_POISON=1 in the environment, every forward fills its
// workspace and residual buffer, and every backward its workspace, with NaN on the stream before
// its kernels run, so a read of memory the kernels did not write reaches the outputs (the
// reference's interpret mode poisons uninitialised scratch the same way)
__global__ void k_poison(uint32_t* p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0x7FC00000u;  // quiet NaN
}

bool poison_on() {
  const char* e = getenv("TJEV_GDN_POISON");
  return e && e[0] == '1';
}

int poison(void* ptr, size_t bytes, void* stream) {
  if (!ptr || bytes < 4) return 0;
  const size_t n = bytes / 4;
  const unsigned grid = (unsigned)std::min<size_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(k_poison, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<uint32_t*>(ptr), n);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : fail(TJEV_GDN_EHIP, std::string("poison fill: ") + hipGetErrorString(e));
}

int poison_buffers(const tjev_gdn_params* p, void* stream, void* workspace, float* residuals, int backward) {
  if (!poison_on()) return 0;
  if (int s = poison(workspace, layout(p, backward).total, stream)) return s;
  return backward ? 0 : poison(residuals, residual_layout(p).total, stream);
}

int run(const tjev_gdn_params* p, void* stream, gdn::GdnArgs& A, int backward) {
  const gdn::ShapeTable* t = lookup(kernel_chunk(p), p->key_dim);
  const gdn::GdnFn fn = t->fn[p->precision][p->io_dtype][p->gate_dtype];
  const hipError_t e = fn(A, static_cast<hipStream_t>(stream), backward, gdn::active_timer());
  if (e != hipSuccess) return fail(TJEV_GDN_EHIP, std::string("HIP launch failed: ") + hipGetErrorString(e));
  return 0;
}

int run_v2(const tjev_gdn_params* p, void* stream, gdn::GdnArgs& A, int backward) {
  const gdn::ShapeTable* t = lookup(kernel_chunk(p), p->key_dim);
  const gdn::GdnFn fn = t->fnv2[p->precision][p->io_dtype][p->qk_dtype][p->gate_dtype];
  const hipError_t e = fn(A, static_cast<hipStream_t>(stream), backward, gdn::active_timer());
  if (e != hipSuccess) return fail(TJEV_GDN_EHIP, std::string("HIP launch failed: ") + hipGetErrorString(e));
  return 0;
}

}  // namespace

namespace gdn {
int fail(int status, const char* msg) { return ::fail(status, msg); }
const Timer* active_timer() { return g_prof.on ? &g_timer : nullptr; }
}  // namespace gdn

extern "C" {

int tjev_gdn_check(const tjev_gdn_params* p) { return validate(p); }

size_t tjev_gdn_states_bytes(const tjev_gdn_params* p) {
  if (validate(p)) return 0;
  const size_t C = kernel_chunk(p);
  const size_t N = (p->length + C - 1) / C;
  return (size_t)p->batch * p->value_heads * N * p->key_dim * p->value_dim * state_elem(p);
}

size_t tjev_gdn_residual_bytes(const tjev_gdn_params* p) {
  if (validate(p)) return 0;
  return residual_layout(p).total;
}

size_t tjev_gdn_workspace_bytes(const tjev_gdn_params* p, int backward) {
  if (validate(p)) return 0;
  return layout(p, backward).total;
}

// the state arguments of a continued sequence, shared by the _cont entry points
int check_state(const tjev_gdn_params* p, const void* initial_state, const void* initial_conv, const void* d_final,
                const void* d_initial_state, const void* d_initial_conv) {
  if (p->taps <= 1 && (initial_conv || d_initial_conv))
    return fail(TJEV_GDN_EINVAL, "a conv history needs a conv of 2 or more taps");
  if (d_initial_conv && !initial_conv)
    return fail(TJEV_GDN_EINVAL, "the conv history's gradient needs the conv history");
  if (d_initial_state && !initial_state)
    return fail(TJEV_GDN_EINVAL, "the initial state's gradient needs the initial state");
  for (const void* q : {initial_state, initial_conv, d_final, d_initial_state, d_initial_conv})
    if (q && !aligned(q, 16)) return fail(TJEV_GDN_EINVAL, "state tensors must be 16-byte aligned");
  return 0;
}

// the megakernel forward, with the gated RMSNorm of its output in the output kernel when y is given
static int mega2_fwd(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
              const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
              const float* initial_state, const void* initial_conv, void* out, float* residuals, float* final_state,
              void* conv_state, const void* gate, const float* norm_weight, float eps, void* y, void* workspace,
              size_t workspace_bytes) {
  if (int s = validate(p)) return s;
  if (y) {
    if (!gate || !norm_weight) return fail(TJEV_GDN_EINVAL, "null tensor argument");
    if (!aligned(gate, 16) || !aligned(y, 16)) return fail(TJEV_GDN_EINVAL, "gate and y must be 16-byte aligned");
    if (!(eps >= 0.f)) return fail(TJEV_GDN_EINVAL, "eps must be >= 0");
  }
  if (!qkv || !a || !b || !a_log || !dt_bias || !seg || !out || !residuals || (p->taps > 0 && !conv_w))
    return fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (!aligned(qkv, 16) || !aligned(out, 16) || !aligned(residuals, 256) || !aligned(workspace, 256))
    return fail(TJEV_GDN_EINVAL, "qkv and out must be 16-byte aligned, the residuals and workspace 256-byte aligned");
  if (int s = check_state(p, initial_state, initial_conv, nullptr, nullptr, nullptr)) return s;
  if (p->taps <= 1 && conv_state) return fail(TJEV_GDN_EINVAL, "a conv history needs a conv of 2 or more taps");
  const Layout L = layout(p, 0);
  if (!workspace || workspace_bytes < L.total)
    return fail(TJEV_GDN_EWORKSPACE, "forward workspace needs " + std::to_string(L.total) + " bytes");
  gdn::GdnArgs A = base_args(p, workspace, L);
  A.qkv = qkv;
  A.ga = a;
  A.gb = b;
  A.a_log = a_log;
  A.dt_bias = dt_bias;
  A.conv_w = conv_w;
  A.seg = seg;
  A.out = out;
  bind_residuals(p, residuals, A);
  A.init_state = initial_state;
  A.init_conv = initial_conv;
  A.final_state = final_state;
  A.conv_state = conv_state;
  A.nz = gate;
  A.nw = norm_weight;
  A.neps = eps;
  A.ny = y;
  if (int s = poison_buffers(p, stream, workspace, residuals, 0)) return s;
  return run(p, stream, A, 0);
}

int tjev_gdn_mega2_fwd_cont(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                            const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                            const float* initial_state, const void* initial_conv, void* out, float* residuals,
                            float* final_state, void* conv_state, void* workspace, size_t workspace_bytes) {
  return mega2_fwd(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, initial_state, initial_conv, out, residuals,
                   final_state, conv_state, nullptr, nullptr, 0.f, nullptr, workspace, workspace_bytes);
}

int tjev_gdn_mega2_fwd_normed(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                              const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                              const float* initial_state, const void* initial_conv, const void* gate,
                              const float* norm_weight, float eps, void* out, void* y, float* residuals,
                              float* final_state, void* conv_state, void* workspace, size_t workspace_bytes) {
  if (!y) return fail(TJEV_GDN_EINVAL, "null tensor argument");
  return mega2_fwd(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, initial_state, initial_conv, out, residuals,
                   final_state, conv_state, gate, norm_weight, eps, y, workspace, workspace_bytes);
}

// The workspace of tjev_gdn_mega2_fwd_cont_noalloc: one array per GPU, held until the process
// ends. Host code uses its per-device address from hipGetSymbolAddress, never the name.
static __device__ __align__(256) char scratch[TJEV_GDN_SCRATCH_BYTES];

// scratch's address on the current device, looked up once per device
int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[64] = {};
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(TJEV_GDN_EHIP, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(TJEV_GDN_EHIP, "device index out of range for the scratch table");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* ptr = nullptr;
    const hipError_t r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (r != hipSuccess || !ptr)
      return fail(TJEV_GDN_EHIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(r));
    addr[dev] = ptr;
  }
  *out = addr[dev];
  return 0;
}

int tjev_gdn_mega2_fwd_cont_noalloc(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                                    const void* b, const float* a_log, const float* dt_bias, const float* conv_w,
                                    const int32_t* seg, const float* initial_state, const void* initial_conv,
                                    void* out, float* residuals, float* final_state, void* conv_state) {
  if (int s = validate(p)) return s;
  const size_t need = layout(p, 0).total;
  if (need > TJEV_GDN_SCRATCH_BYTES)
    return fail(TJEV_GDN_EWORKSPACE, "the forward needs " + std::to_string(need) + " bytes of workspace, more than the " +
                                         std::to_string((size_t)TJEV_GDN_SCRATCH_BYTES) +
                                         " of the static scratch: use tjev_gdn_mega2_fwd_cont");
  void* ws = nullptr;
  if (int s = scratch_address(&ws)) return s;
  return tjev_gdn_mega2_fwd_cont(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, initial_state, initial_conv, out,
                                 residuals, final_state, conv_state, ws, TJEV_GDN_SCRATCH_BYTES);
}

int tjev_gdn_mega2_fwd(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                       const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg, void* out,
                       float* residuals, void* workspace, size_t workspace_bytes) {
  return tjev_gdn_mega2_fwd_cont(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, nullptr, nullptr, out, residuals,
                                 nullptr, nullptr, workspace, workspace_bytes);
}

int tjev_gdn_mega2_fwd_state(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                             const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                             void* out, float* residuals, float* final_state, void* conv_state, void* workspace,
                             size_t workspace_bytes) {
  return tjev_gdn_mega2_fwd_cont(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, nullptr, nullptr, out, residuals,
                                 final_state, conv_state, workspace, workspace_bytes);
}

int tjev_gdn_v2_fwd_cont(const tjev_gdn_params* p, void* stream, const void* q, const void* k, const void* v,
                         const void* g, const void* beta, const int32_t* seg, const float* initial_state, void* out,
                         float* residuals, float* final_state, void* workspace, size_t workspace_bytes) {
  if (int s = validate(p)) return s;
  if (p->taps != 0) return fail(TJEV_GDN_EINVAL, "the v2 operator has no conv: taps must be 0");
  if (!q || !k || !v || !g || !beta || !seg || !out || !residuals) return fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(out, 16) || !aligned(residuals, 256) ||
      !aligned(workspace, 256))
    return fail(TJEV_GDN_EINVAL, "q, k, v and out must be 16-byte aligned, the residuals and workspace 256-byte aligned");
  if (int s = check_state(p, initial_state, nullptr, nullptr, nullptr, nullptr)) return s;
  const Layout L = layout(p, 0);
  if (!workspace || workspace_bytes < L.total)
    return fail(TJEV_GDN_EWORKSPACE, "forward workspace needs " + std::to_string(L.total) + " bytes");
  gdn::GdnArgs A = base_args(p, workspace, L);
  A.q2 = q;
  A.k2 = k;
  A.v2 = v;
  A.g2 = g;
  A.b2 = beta;
  A.seg = seg;
  A.out = out;
  bind_residuals(p, residuals, A);
  A.init_state = initial_state;
  A.final_state = final_state;
  if (int s = poison_buffers(p, stream, workspace, residuals, 0)) return s;
  return run_v2(p, stream, A, 0);
}

int tjev_gdn_v2_fwd(const tjev_gdn_params* p, void* stream, const void* q, const void* k, const void* v,
                    const void* g, const void* beta, const int32_t* seg, void* out, float* residuals, void* workspace,
                    size_t workspace_bytes) {
  return tjev_gdn_v2_fwd_cont(p, stream, q, k, v, g, beta, seg, nullptr, out, residuals, nullptr, workspace,
                              workspace_bytes);
}

int tjev_gdn_v2_bwd_cont(const tjev_gdn_params* p, void* stream, const void* q, const void* k, const void* v,
                         const void* g, const void* beta, const int32_t* seg, const float* initial_state,
                         const float* residuals, const void* d_out, const float* d_final_state, void* d_q, void* d_k,
                         void* d_v, void* d_g, void* d_beta, float* d_initial_state, void* workspace,
                         size_t workspace_bytes) {
  if (int s = validate(p)) return s;
  if (p->taps != 0) return fail(TJEV_GDN_EINVAL, "the v2 operator has no conv: taps must be 0");
  if (!q || !k || !v || !g || !beta || !seg || !residuals || !d_out || !d_q || !d_k || !d_v || !d_g || !d_beta)
    return fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(d_out, 16) || !aligned(d_q, 16) ||
      !aligned(d_k, 16) || !aligned(d_v, 16) || !aligned(residuals, 256) || !aligned(workspace, 256))
    return fail(TJEV_GDN_EINVAL, "tensors must be 16-byte aligned, the residuals and workspace 256-byte aligned");
  if (int s = check_state(p, initial_state, nullptr, d_final_state, d_initial_state, nullptr)) return s;
  const Layout L = layout(p, 1);
  if (!workspace || workspace_bytes < L.total)
    return fail(TJEV_GDN_EWORKSPACE, "backward workspace needs " + std::to_string(L.total) + " bytes");
  gdn::GdnArgs A = base_args(p, workspace, L);
  A.q2 = q;
  A.k2 = k;
  A.v2 = v;
  A.g2 = g;
  A.b2 = beta;
  A.seg = seg;
  bind_residuals(p, const_cast<float*>(residuals), A);
  A.d_out = d_out;
  A.d_q2 = d_q;
  A.d_k2 = d_k;
  A.d_v2 = d_v;
  A.d_g2 = d_g;
  A.d_b2 = d_beta;
  A.init_state = initial_state;
  A.d_final = d_final_state;
  A.d_init_state = d_initial_state;
  if (int s = poison_buffers(p, stream, workspace, nullptr, 1)) return s;
  return run_v2(p, stream, A, 1);
}

int tjev_gdn_v2_bwd(const tjev_gdn_params* p, void* stream, const void* q, const void* k, const void* v,
                    const void* g, const void* beta, const int32_t* seg, const float* residuals, const void* d_out,
                    void* d_q, void* d_k, void* d_v, void* d_g, void* d_beta, void* workspace,
                    size_t workspace_bytes) {
  return tjev_gdn_v2_bwd_cont(p, stream, q, k, v, g, beta, seg, nullptr, residuals, d_out, nullptr, d_q, d_k, d_v, d_g,
                              d_beta, nullptr, workspace, workspace_bytes);
}

// The gated RMSNorm's backward ahead of the megakernel's (tjev_gdn_mega2_bwd_normed): its
// inputs, and where its d out goes (a part of the caller's workspace).
struct NormBwd {
  const void* out;
  const void* gate;
  const float* weight;
  float eps;
  const void* d_y;
  void* d_gate;
  float* d_weight;
};

// the extra workspace of tjev_gdn_mega2_bwd_normed after the megakernel backward's: d out, then
// the norm's weight-gradient partials
static size_t norm_bwd_extra(const tjev_gdn_params* p, int weight_grad, tjev_gdn_norm_params* np, size_t* dout_bytes) {
  np->tokens = (int64_t)p->batch * p->length;
  np->heads = p->value_heads;
  np->dim = p->value_dim;
  np->dtype = p->io_dtype;
  np->eps = 0.f;
  *dout_bytes = ((size_t)np->tokens * p->value_heads * p->value_dim * (p->io_dtype == TJEV_GDN_BF16 ? 2 : 4) + 255) &
                ~size_t(255);
  return *dout_bytes + tjev_gdn_norm_workspace_bytes(np, weight_grad);
}

static int mega2_bwd(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                     const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                     const float* initial_state, const void* initial_conv, const float* residuals, const void* d_out,
                     const float* d_final_state, void* d_qkv, void* d_a, void* d_b, float* d_a_log, float* d_dt_bias,
                     float* d_conv_w, float* d_initial_state, void* d_initial_conv, void* workspace,
                     size_t workspace_bytes, const NormBwd* nb) {
  if (int s = validate(p)) return s;
  if (nb) {  // d out comes from the norm's backward, into the workspace after the megakernel's part
    if (!nb->out || !nb->gate || !nb->weight || !nb->d_y || !nb->d_gate) return fail(TJEV_GDN_EINVAL, "null tensor argument");
    if (!aligned(nb->out, 16) || !aligned(nb->gate, 16) || !aligned(nb->d_y, 16) || !aligned(nb->d_gate, 16))
      return fail(TJEV_GDN_EINVAL, "out, gate, d_y and d_gate must be 16-byte aligned");
    if (!(nb->eps >= 0.f)) return fail(TJEV_GDN_EINVAL, "eps must be >= 0");
    d_out = workspace ? static_cast<char*>(workspace) + layout(p, 1).total : nullptr;
  }
  if (!qkv || !a || !b || !a_log || !dt_bias || !seg || !residuals || (!d_out && !nb) || !d_qkv || !d_a || !d_b ||
      !d_a_log || !d_dt_bias || (p->taps > 0 && !conv_w))
    return fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (p->taps == 0 && d_conv_w) return fail(TJEV_GDN_EINVAL, "no conv weight gradient without a conv (taps == 0)");
  if (!aligned(qkv, 16) || !aligned(d_out, 16) || !aligned(d_qkv, 16) || !aligned(residuals, 256) ||
      !aligned(workspace, 256))
    return fail(TJEV_GDN_EINVAL, "tensors must be 16-byte aligned, the residuals and workspace 256-byte aligned");
  if (int s = check_state(p, initial_state, initial_conv, d_final_state, d_initial_state, d_initial_conv)) return s;
  const Layout L = layout(p, 1);
  tjev_gdn_norm_params np{};
  size_t dout_bytes = 0;
  const size_t need = L.total + (nb ? norm_bwd_extra(p, nb->d_weight != nullptr, &np, &dout_bytes) : 0);
  if (!workspace || workspace_bytes < need)
    return fail(TJEV_GDN_EWORKSPACE, "backward workspace needs " + std::to_string(need) + " bytes");
  gdn::GdnArgs A = base_args(p, workspace, L);
  A.qkv = qkv;
  A.ga = a;
  A.gb = b;
  A.a_log = a_log;
  A.dt_bias = dt_bias;
  A.conv_w = conv_w;
  A.seg = seg;
  bind_residuals(p, const_cast<float*>(residuals), A);
  A.d_out = d_out;
  A.d_qkv = d_qkv;
  A.d_a = d_a;
  A.d_b = d_b;
  A.d_a_log = d_a_log;
  A.d_dt_bias = d_dt_bias;
  A.d_conv_w = d_conv_w;
  A.init_state = initial_state;
  A.init_conv = initial_conv;
  A.d_final = d_final_state;
  A.d_init_state = d_initial_state;
  A.d_init_conv = d_initial_conv;
  // the poison mode fills the whole workspace: with the norm, its d out and weight partials too
  if (poison_on())
    if (int s = poison(workspace, need, stream)) return s;
  if (!nb) return run(p, stream, A, 1);
  // the norm's backward into d out, then the megakernel's, on the caller's stream
  np.eps = nb->eps;
  char* nws = static_cast<char*>(workspace) + L.total + dout_bytes;
  if (int s = tjev_gdn_gated_rmsnorm_bwd(&np, stream, nb->out, nb->gate, nb->weight, seg, nb->d_y,
                                         const_cast<void*>(d_out), nb->d_gate, nb->d_weight, nws,
                                         workspace_bytes - L.total - dout_bytes))
    return s;
  return run(p, stream, A, 1);
}

int tjev_gdn_mega2_bwd_cont(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                            const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                            const float* initial_state, const void* initial_conv, const float* residuals,
                            const void* d_out, const float* d_final_state, void* d_qkv, void* d_a, void* d_b,
                            float* d_a_log, float* d_dt_bias, float* d_conv_w, float* d_initial_state,
                            void* d_initial_conv, void* workspace, size_t workspace_bytes) {
  return mega2_bwd(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, initial_state, initial_conv, residuals, d_out,
                   d_final_state, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_conv_w, d_initial_state, d_initial_conv,
                   workspace, workspace_bytes, nullptr);
}

size_t tjev_gdn_workspace_bytes_normed(const tjev_gdn_params* p, int norm_weight_grad) {
  if (validate(p)) return 0;
  tjev_gdn_norm_params np{};
  size_t dout_bytes = 0;
  return layout(p, 1).total + norm_bwd_extra(p, norm_weight_grad, &np, &dout_bytes);
}

int tjev_gdn_mega2_bwd_normed(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                              const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                              const float* initial_state, const void* initial_conv, const float* residuals,
                              const void* out, const void* gate, const float* norm_weight, float eps, const void* d_y,
                              const float* d_final_state, void* d_qkv, void* d_a, void* d_b, float* d_a_log,
                              float* d_dt_bias, float* d_conv_w, float* d_initial_state, void* d_initial_conv,
                              void* d_gate, float* d_norm_weight, void* workspace, size_t workspace_bytes) {
  const NormBwd nb{out, gate, norm_weight, eps, d_y, d_gate, d_norm_weight};
  return mega2_bwd(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, initial_state, initial_conv, residuals, nullptr,
                   d_final_state, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_conv_w, d_initial_state, d_initial_conv,
                   workspace, workspace_bytes, &nb);
}

int tjev_gdn_mega2_bwd(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a, const void* b,
                       const float* a_log, const float* dt_bias, const float* conv_w, const int32_t* seg,
                       const float* residuals, const void* d_out, void* d_qkv, void* d_a, void* d_b, float* d_a_log,
                       float* d_dt_bias, float* d_conv_w, void* workspace, size_t workspace_bytes) {
  return tjev_gdn_mega2_bwd_cont(p, stream, qkv, a, b, a_log, dt_bias, conv_w, seg, nullptr, nullptr, residuals, d_out,
                                 nullptr, d_qkv, d_a, d_b, d_a_log, d_dt_bias, d_conv_w, nullptr, nullptr, workspace,
                                 workspace_bytes);
}

int tjev_gdn_profile_begin(void) {
  g_prof.on = true;
  return 0;
}

int tjev_gdn_profile_end(float* ms, int* launches, int n) {
  g_prof.on = false;
  for (int k = 0; k < n; ++k) {
    ms[k] = 0.f;
    launches[k] = 0;
  }
  int status = 0;
  if (g_prof.err != hipSuccess) status = fail(TJEV_GDN_EHIP, std::string("profiling: ") + hipGetErrorString(g_prof.err));
  for (auto& m : g_prof.marks) {
    float t = 0.f;
    if (hipEventSynchronize(m.second.second) == hipSuccess &&
        hipEventElapsedTime(&t, m.second.first, m.second.second) == hipSuccess && m.first < n) {
      ms[m.first] += t;
      launches[m.first] += 1;
    }
    g_prof.pool.push_back(m.second.first);
    g_prof.pool.push_back(m.second.second);
  }
  g_prof.marks.clear();
  g_prof.err = hipSuccess;
  return status;
}

const char* tjev_gdn_kernel_name(int kernel) {
  return (kernel >= 0 && kernel < gdn::K_COUNT) ? kKernelNames[kernel] : "";
}

const char* tjev_gdn_last_error(void) { return g_error.c_str(); }

int tjev_gdn_version(void) { return (0 << 16) | 1; }

int tjev_gdn_lds_poison(void) {
#ifdef GDN_LDS_POISON
  return 1;
#else
  return 0;
#endif
}

}  // extern "C"
