// One decode step of the GDN layer core for gfx950: T = 1 new token per row, continuing the
// conv history and the recurrent state left by the prefill (or by the previous step). It is
// the token recurrence of xla.py:141-167 (the reference's "T=1 decode step") on the
// megakernel's inputs, with the conv over the K-1 kept raw rows and the new one (HF
// causal_conv1d_update), SiLU, the q/k l2norm and the gates as k_prep computes them.
//
// One workgroup per (row, value head, tile of tile_cols<D>() value columns: the whole head, one
// q and k build per head): it rebuilds its q and k head and its v columns from the raw rows,
// then updates its D x tile slice of the state: s = s e^g, delta = (v - s^T k) beta,
// s += k delta^T, o = s^T q. Each thread holds 4 adjacent columns of several rows (16-byte
// accesses); the two column sums go through lane shuffles and LDS. The state is read and
// written once (in place allowed: each slice belongs to one workgroup); the new conv history
// goes to a separate buffer, copied in 16-byte pieces by all the workgroups of each row.
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/tjev_gdn.h"
#include "gdn_device.h"
#include "gdn_launch.h"

namespace gdn {
namespace {

struct DecodeArgs {
  int B, Hk, H, ratio, taps, W;
  float scale;
  const void* qkv;       // [B, W] the new raw row
  const void* ga;        // [B, H]
  const void* gb;        // [B, H]
  const float* a_log;    // [H]
  const float* dt_bias;  // [H]
  const float* conv_w;   // [K, W]
  const void* conv_in;   // [B, K-1, W] the raw rows before it, oldest first
  const float* state;    // [B, H, Dk, Dv]
  void* out;             // [B, H, Dv]
  void* conv_out;        // [B, K-1, W]
  float* state_out;      // [B, H, Dk, Dv]
};

constexpr int kThreads = 256;
typedef float v4f __attribute__((ext_vector_type(4)));  // the nontemporal builtins' vector type
// value columns per workgroup: the whole head (measured at the 0.8B heads, 64 rows: 27.5-28.9
// against 29.4-30.2 us per step with tiles of 32, 28.2-28.7 with 64, 46 with 16; 512 threads
// per workgroup with whole heads: no faster)
template <int D>
constexpr int tile_cols() { return D; }

// channel c's raw values for its activation: the new row and the K-1 kept rows with their conv
// weights, loaded as soon as the workgroup starts
template <class TIO>
struct TapRow {
  float x[5], w[5];  // x[L] = x[t - L], w[L] = w[K-1-L]
  __device__ __forceinline__ void fetch(const DecodeArgs& A, int b, int c) {
    x[0] = ldf(reinterpret_cast<const TIO*>(A.qkv) + (size_t)b * A.W + c);
    if (A.taps == 0) return;
    const TIO* hist = reinterpret_cast<const TIO*>(A.conv_in) + (size_t)b * (A.taps - 1) * A.W;
    w[0] = A.conv_w[(size_t)(A.taps - 1) * A.W + c];
#pragma unroll
    for (int L = 1; L < 5; ++L) {
      if (L < A.taps) {
        x[L] = ldf(hist + (size_t)(A.taps - 1 - L) * A.W + c);
        w[L] = A.conv_w[(size_t)(A.taps - 1 - L) * A.W + c];
      }
    }
  }
  // the causal conv, lag 0 first (causal_conv1d.py:42-45), then SiLU; the new row itself
  // without a conv (taps == 0)
  __device__ __forceinline__ float act(const DecodeArgs& A) const {
    if (A.taps == 0) return x[0];
    float z = x[0] * w[0];
#pragma unroll
    for (int L = 1; L < 5; ++L)
      if (L < A.taps) z += x[L] * w[L];
    return z * sigmoid_io<TIO>(z);
  }
};

// the block sums of two values per thread (wave sums, then the waves in order)
__device__ __forceinline__ float2 block_sum2(float a, float b, float (*red)[kThreads / 64]) {
  a = sum64(a);
  b = sum64(b);
  if (lane() == 0) {
    red[0][wave()] = a;
    red[1][wave()] = b;
  }
  __syncthreads();
  float2 s = make_float2(0.f, 0.f);
#pragma unroll
  for (int q = 0; q < kThreads / 64; ++q) {
    s.x += red[0][q];
    s.y += red[1][q];
  }
  return s;
}

template <int D, class TIO, class TG>
__global__ __launch_bounds__(kThreads) void k_decode(DecodeArgs A) {
  constexpr int DT = tile_cols<D>();
  constexpr int NTL = D / DT;
  constexpr int QPR = DT / 4;                 // column quads of a tile (one per thread)
  constexpr int RG = kThreads / QPR;          // row groups
  constexpr int RPT = (D + RG - 1) / RG;      // rows per thread
  __shared__ float sq[D], sk[D], sv[DT];
  __shared__ float red[2][kThreads / 64];
  __shared__ float part[2][kThreads / 64][DT];  // one buffer per column sum: no barrier before a write
  __shared__ float gate[2];
  const int tile = blockIdx.x % NTL, bh = blockIdx.x / NTL, h = bh % A.H, b = bh / A.H, hk = h / A.ratio;
  const int tid = threadIdx.x;
  const int cq = tid % QPR, rg = tid / QPR, c0 = 4 * cq;
  // the activations' raw inputs and the gates first, then the state slice (16-byte loads):
  // memory operations complete in issue order, so building q, k and v waits only for the
  // former while the state's loads are still in flight
  TapRow<TIO> tq, tk, tv;
  if (tid < D) {
    tq.fetch(A, b, hk * D + tid);
    tk.fetch(A, b, A.Hk * D + hk * D + tid);
  }
  if (tid < DT) tv.fetch(A, b, 2 * A.Hk * D + h * D + tile * DT + tid);
  float av = 0.f, bv = 0.f, alog = 0.f, dtb = 0.f;
  if (tid == 0) {
    av = ldf(reinterpret_cast<const TG*>(A.ga) + (size_t)b * A.H + h);
    bv = ldf(reinterpret_cast<const TG*>(A.gb) + (size_t)b * A.H + h);
    alog = A.a_log[h];
    dtb = A.dt_bias[h];
  }
  const float* src = A.state + (size_t)bh * D * D + tile * DT + c0;
  float4 s[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg * RPT + r;
    // the state streams through once: nontemporal loads and stores (27.3-28.1 against 28.5-30.1 us
    // per kernel at 64 rows of the 0.8B heads)
    const v4f t = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(src + (size_t)(i < D ? i : D - 1) * D));
    s[r] = make_float4(t.x, t.y, t.z, t.w);
  }
  // q and k of key head hk, v of value head h (this tile's columns)
  const float aq = tid < D ? tq.act(A) : 0.f;
  const float ak = tid < D ? tk.act(A) : 0.f;
  if (tid < DT) sv[tid] = tv.act(A);
  if (tid == 0) {  // beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias)
    gate[0] = sigmoidf_(bv);
    gate[1] = expf(-expf(alog) * softplusf_(av + dtb));
  }
  // l2norm (xla.py:42-53; r = 0 on an all-zero row), q scaled by Dk^-1/2
  const float2 ss = block_sum2(aq * aq, ak * ak, red);
  const float rq = (ss.x == 0.f ? 0.f : 1.0f / sqrtf(ss.x + 1e-6f)) * A.scale;
  const float rk = ss.y == 0.f ? 0.f : 1.0f / sqrtf(ss.y + 1e-6f);
  if (tid < D) {
    sq[tid] = aq * rq;
    sk[tid] = ak * rk;
  }
  __syncthreads();
  // column sums over the rows: within the thread, across the wave's row groups (xor
  // shuffles over the lanes of one column quad), then across the waves through LDS
  auto column_sums = [&](int k, float4 v, float (&out)[4]) {
    float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int m = QPR; m < 64; m <<= 1)
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] += __shfl_xor(x[e], m);
    if (lane() < QPR) {
#pragma unroll
      for (int e = 0; e < 4; ++e) part[k][wave()][c0 + e] = x[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float t = 0.f;
#pragma unroll
      for (int q = 0; q < kThreads / 64; ++q) t += part[k][q][c0 + e];
      out[e] = t;
    }
  };
  const float decay = gate[1];
  float4 mem = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg * RPT + r;
    const float kv = i < D ? sk[i] : 0.f;
    s[r].x *= decay; s[r].y *= decay; s[r].z *= decay; s[r].w *= decay;
    mem.x += s[r].x * kv; mem.y += s[r].y * kv; mem.z += s[r].z * kv; mem.w += s[r].w * kv;
  }
  float m[4];
  column_sums(0, mem, m);
  const float bt = gate[0];
  const float dl[4] = {(sv[c0] - m[0]) * bt, (sv[c0 + 1] - m[1]) * bt, (sv[c0 + 2] - m[2]) * bt,
                       (sv[c0 + 3] - m[3]) * bt};
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  float* dst = A.state_out + (size_t)bh * D * D + tile * DT + c0;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg * RPT + r;
    if (i < D) {
      const float kv = sk[i], qv = sq[i];
      s[r].x += kv * dl[0]; s[r].y += kv * dl[1]; s[r].z += kv * dl[2]; s[r].w += kv * dl[3];
      o.x += s[r].x * qv; o.y += s[r].y * qv; o.z += s[r].z * qv; o.w += s[r].w * qv;
      const v4f t = {s[r].x, s[r].y, s[r].z, s[r].w};
      __builtin_nontemporal_store(t, reinterpret_cast<v4f*>(dst + (size_t)i * D));
    }
  }
  float ov[4];
  column_sums(1, o, ov);
  if (rg == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) stf(reinterpret_cast<TIO*>(A.out) + (size_t)bh * D + tile * DT + c0 + e, ov[e]);
  }
  if (A.taps > 1) {  // the history shifted by the new row, in 16-byte pieces spread over the row's workgroups
    constexpr int E = 16 / sizeof(TIO);
    const int k1 = A.taps - 1, wu = A.W / E, units = k1 * wu;
    const uint4* hist = reinterpret_cast<const uint4*>(reinterpret_cast<const TIO*>(A.conv_in) + (size_t)b * k1 * A.W);
    const uint4* x = reinterpret_cast<const uint4*>(reinterpret_cast<const TIO*>(A.qkv) + (size_t)b * A.W);
    uint4* out = reinterpret_cast<uint4*>(reinterpret_cast<TIO*>(A.conv_out) + (size_t)b * k1 * A.W);
    for (int u = (h * NTL + tile) * kThreads + tid; u < units; u += A.H * NTL * kThreads) {
      const int r = u / wu, c = u % wu;
      out[u] = r + 1 < k1 ? hist[(size_t)(r + 1) * wu + c] : x[c];
    }
  }
}

template <int D>
hipError_t launch(const DecodeArgs& A, int io, int gate, hipStream_t st) {
  const dim3 grid(A.B * A.H * (D / tile_cols<D>()));
  if (io == TJEV_GDN_BF16 && gate == TJEV_GDN_BF16) hipLaunchKernelGGL((k_decode<D, uint16_t, uint16_t>), grid, dim3(kThreads), 0, st, A);
  if (io == TJEV_GDN_BF16 && gate == TJEV_GDN_F32) hipLaunchKernelGGL((k_decode<D, uint16_t, float>), grid, dim3(kThreads), 0, st, A);
  if (io == TJEV_GDN_F32 && gate == TJEV_GDN_BF16) hipLaunchKernelGGL((k_decode<D, float, uint16_t>), grid, dim3(kThreads), 0, st, A);
  if (io == TJEV_GDN_F32 && gate == TJEV_GDN_F32) hipLaunchKernelGGL((k_decode<D, float, float>), grid, dim3(kThreads), 0, st, A);
  return hipGetLastError();
}

}  // namespace
}  // namespace gdn

extern "C" int tjev_gdn_decode_step(const tjev_gdn_params* p, void* stream, const void* qkv, const void* a,
                                    const void* b, const float* a_log, const float* dt_bias, const float* conv_w,
                                    const void* conv_state, const float* state, void* out, void* conv_state_out,
                                    float* state_out) {
  auto fail = [](int status, const std::string& msg) { return gdn::fail(status, msg.c_str()); };
  if (!p) return fail(TJEV_GDN_EINVAL, "null params");
  if (p->batch <= 0 || p->key_heads <= 0 || p->value_heads <= 0)
    return fail(TJEV_GDN_EINVAL, "batch and head counts must be positive");
  if (p->length != 1) return fail(TJEV_GDN_EINVAL, "a decode step takes one token per row (length 1)");
  if (p->value_heads % p->key_heads)
    return fail(TJEV_GDN_EINVAL, std::to_string(p->value_heads) + " value heads are not groups of " +
                                     std::to_string(p->key_heads) + " key heads");
  if (p->key_dim != p->value_dim) return fail(TJEV_GDN_EUNSUPPORTED, "this build's kernels need key_dim == value_dim");
  const int D = p->key_dim;
  if (D != 16 && D != 32 && D != 64 && D != 128)
    return fail(TJEV_GDN_EUNSUPPORTED, "decode kernels exist for head dims 16, 32, 64 and 128");
  if (p->taps < 0 || p->taps > 5) return fail(TJEV_GDN_EINVAL, "conv kernel of " + std::to_string(p->taps) + " taps: 1..5");
  if (p->io_dtype < 0 || p->io_dtype > 1 || p->gate_dtype < 0 || p->gate_dtype > 1)
    return fail(TJEV_GDN_EINVAL, "dtypes must be TJEV_GDN_F32 or TJEV_GDN_BF16");
  if (!qkv || !a || !b || !a_log || !dt_bias || !state || !out || !state_out ||
      (p->taps > 0 && !conv_w) || (p->taps > 1 && (!conv_state || !conv_state_out)))
    return fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (p->taps > 1 && conv_state == conv_state_out)
    return fail(TJEV_GDN_EINVAL, "conv_state_out must not alias conv_state (every head reads the history)");
  auto al16 = [](const void* q) { return q == nullptr || (reinterpret_cast<uintptr_t>(q) % 16) == 0; };
  if (!al16(qkv) || !al16(state) || !al16(state_out) || (p->taps > 1 && (!al16(conv_state) || !al16(conv_state_out))))
    return fail(TJEV_GDN_EINVAL, "qkv, the conv states and the states must be 16-byte aligned");
  gdn::DecodeArgs A{};
  A.B = p->batch;
  A.Hk = p->key_heads;
  A.H = p->value_heads;
  A.ratio = p->value_heads / p->key_heads;
  A.taps = p->taps;
  A.W = 2 * p->key_heads * D + p->value_heads * D;
  A.scale = 1.0f / sqrtf((float)D);
  A.qkv = qkv;
  A.ga = a;
  A.gb = b;
  A.a_log = a_log;
  A.dt_bias = dt_bias;
  A.conv_w = conv_w;
  A.conv_in = conv_state;
  A.state = state;
  A.out = out;
  A.conv_out = conv_state_out;
  A.state_out = state_out;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const gdn::Timer* tm = gdn::active_timer();
  if (tm) tm->mark(tm->self, gdn::K_DECODE, 0, st);
  hipError_t e = hipSuccess;
  switch (D) {
    case 16: e = gdn::launch<16>(A, p->io_dtype, p->gate_dtype, st); break;
    case 32: e = gdn::launch<32>(A, p->io_dtype, p->gate_dtype, st); break;
    case 64: e = gdn::launch<64>(A, p->io_dtype, p->gate_dtype, st); break;
    default: e = gdn::launch<128>(A, p->io_dtype, p->gate_dtype, st); break;
  }
  if (tm) tm->mark(tm->self, gdn::K_DECODE, 1, st);
  if (e != hipSuccess) return fail(TJEV_GDN_EHIP, std::string("HIP launch failed: ") + hipGetErrorString(e));
  return 0;
}
