// The gated RMSNorm of the GDN output (tjev's GatedRMSNorm, src/tjev/model/norms.py:13-15,
// 36-62, with the padding select of src/tjev/model/gdn.py:157-163) and its backward, for gfx950.
//
// HBM-bound: one (token, head) row of D values per group of D/8 lanes, 8 consecutive values per
// lane (one 16-byte bf16 or two 16-byte fp32 loads); the row's sums of squares and of dn * n
// are lane-group reductions by xor shuffles. The backward runs a fixed grid that strides over
// the rows so that each workgroup's weight-gradient partial is a fixed-order sum; the partials
// are added in fp64 by a second kernel.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "../../include/tjev_gdn.h"
#include "gdn_device.h"
#include "gdn_launch.h"

namespace gdn {
namespace {

struct NormArgs {
  long rows;  // tokens * heads
  int heads;
  float eps;
  const void* x;
  const void* z;
  const float* w;
  const int32_t* seg;
  const void* dy;
  void* y;
  void* dx;
  void* dz;
  float* dwp;  // [gridDim.x, D] partials, or null
  float* dw;
  int nblk;
};

constexpr int kThreads = 256;
constexpr int kMaxBwdBlocks = 2048;
constexpr int kFwdRows = 2;  // rows per lane group in the forward (measured: 4 and 8 are slower)

// round to the storage type and back (what astype(dtype).astype(float32) does)
template <class T>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (std::is_same<T, uint16_t>::value) {
    return bf2f(f2bf(v));
  } else {
    return v;
  }
}

__device__ __forceinline__ void st8(float* p, const float (&v)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void st8(uint16_t* p, const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = (uint32_t)f2bf(v[2 * e]) | ((uint32_t)f2bf(v[2 * e + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}

// sum over the LPR lanes of one row (groups of LPR consecutive lanes, LPR a power of two)
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  return sum_lanes<LPR>(v);
}

template <class T>
__device__ __forceinline__ void load_row(const void* base, long row, int D, int c0, bool live, float (&v)[8]) {
  if (live) {
    ld8(static_cast<const T*>(base) + row * D + c0, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
  }
}

// y = w * rnd(x * rsqrt(mean x^2 + eps)) * silu(z), 0 on padding tokens (norms.py:13-15, 36-40).
// Each lane group takes kFwdRows rows spaced one workgroup-tile apart, every load issued first.
template <int D, class T>
__global__ __launch_bounds__(kThreads) void k_norm_fwd(NormArgs A) {
  constexpr int LPR = D / 8, RPB = kThreads / LPR, R = kFwdRows;
  const int c0 = (threadIdx.x % LPR) * 8;
  const long row0 = (long)blockIdx.x * RPB * R + threadIdx.x / LPR;
  float x[R][8], z[R][8];
  int sg[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const long row = row0 + (long)i * RPB;
    load_row<T>(A.x, row, D, c0, row < A.rows, x[i]);
    load_row<T>(A.z, row, D, c0, row < A.rows, z[i]);
    sg[i] = (A.seg && row < A.rows) ? A.seg[row / A.heads] : 1;
  }
  float w[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) w[e] = A.w[c0 + e];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const long row = row0 + (long)i * RPB;
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[i][e] * x[i][e];
    ss = group_sum<LPR>(ss);
    const float r = rsqrt_io<T>(ss * (1.0f / D) + A.eps);
    const bool valid = sg[i] > 0;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = valid ? w[e] * rnd<T>(x[i][e] * r) * (z[i][e] * sigmoid_io<T>(z[i][e])) : 0.f;
    if (row < A.rows) st8(static_cast<T*>(A.y) + row * D + c0, y);
  }
}

// With n = x r, r = rsqrt(mean x^2 + eps), n^ = rnd(n), s = silu(z), g = dy (0 on padding):
//   dn = rnd(g w s)         (the cotangent of the rounding cast, rounded as autodiff does)
//   dz = g w n^ s'(z)       s'(z) = sig(z) (1 + z (1 - sig(z)))
//   dx = r (dn - n sum(dn n) / D)
//   dw = sum over rows of g n^ s
template <int D, class T>
__global__ __launch_bounds__(kThreads) void k_norm_bwd(NormArgs A) {
  constexpr int LPR = D / 8, RPB = kThreads / LPR;
  __shared__ float sdw[RPB][D];
  const int c0 = (threadIdx.x % LPR) * 8;
  float w[8], dwacc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    w[e] = A.w[c0 + e];
    dwacc[e] = 0.f;
  }
  constexpr int R = 1;  // rows per lane group per iteration (more cost occupancy)
  for (long base = (long)blockIdx.x * RPB * R; base < A.rows; base += (long)gridDim.x * RPB * R) {
    float x[R][8], z[R][8], g[R][8];
    bool valid[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const long row = base + (long)i * RPB + threadIdx.x / LPR;
      const bool live = row < A.rows;
      load_row<T>(A.x, row, D, c0, live, x[i]);
      load_row<T>(A.z, row, D, c0, live, z[i]);
      load_row<T>(A.dy, row, D, c0, live, g[i]);
      valid[i] = live && (!A.seg || A.seg[row / A.heads] > 0);
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const long row = base + (long)i * RPB + threadIdx.x / LPR;
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x[i][e] * x[i][e];
      ss = group_sum<LPR>(ss);
      const float r = rsqrt_io<T>(ss * (1.0f / D) + A.eps);
      float n[8], dn[8], dzv[8], dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float ge = valid[i] ? g[i][e] : 0.f;
        const float sg = sigmoid_io<T>(z[i][e]);
        const float s = z[i][e] * sg;
        n[e] = x[i][e] * r;
        const float nh = rnd<T>(n[e]);
        dn[e] = rnd<T>(ge * w[e] * s);
        dzv[e] = ge * w[e] * nh * (sg * (1.f + z[i][e] * (1.f - sg)));
        dwacc[e] += ge * nh * s;
        dot += dn[e] * n[e];
      }
      dot = group_sum<LPR>(dot) * (1.0f / D);
      float dxv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) dxv[e] = r * (dn[e] - n[e] * dot);
      if (row < A.rows) {
        st8(static_cast<T*>(A.dx) + row * D + c0, dxv);
        st8(static_cast<T*>(A.dz) + row * D + c0, dzv);
      }
    }
  }
  if (!A.dwp) return;
#pragma unroll
  for (int e = 0; e < 8; ++e) sdw[threadIdx.x / LPR][c0 + e] = dwacc[e];
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += kThreads) {
    float s = 0.f;
    for (int q = 0; q < RPB; ++q) s += sdw[q][d];
    A.dwp[(size_t)blockIdx.x * D + d] = s;
  }
}

// d_weight[d] = sum over the backward's workgroups of their partials, in fp64, fixed order
__global__ __launch_bounds__(kThreads) void k_norm_reduce(NormArgs A, int D) {
  const int d = blockIdx.x * kThreads + threadIdx.x;
  if (d >= D) return;
  double s = 0.0;
  for (int b = 0; b < A.nblk; ++b) s += (double)A.dwp[(size_t)b * D + d];
  A.dw[d] = (float)s;
}

template <int D, class T>
hipError_t launch(const NormArgs& A, hipStream_t st, int backward) {
  constexpr int RPB = kThreads / (D / 8);
  const long blocks = (A.rows + RPB * kFwdRows - 1) / (RPB * kFwdRows);
  const Timer* tm = active_timer();
  auto mark = [&](int k, int end) {
    if (tm) tm->mark(tm->self, k, end, st);
  };
  if (!backward) {
    mark(K_NORM_FWD, 0);
    hipLaunchKernelGGL((k_norm_fwd<D, T>), dim3((unsigned)blocks), dim3(kThreads), 0, st, A);
    mark(K_NORM_FWD, 1);
  } else {
    if (A.nblk > 0) {
      mark(K_NORM_BWD, 0);
      hipLaunchKernelGGL((k_norm_bwd<D, T>), dim3((unsigned)A.nblk), dim3(kThreads), 0, st, A);
      mark(K_NORM_BWD, 1);
    }
    if (A.dwp) {
      mark(K_NORM_REDUCE, 0);
      hipLaunchKernelGGL(k_norm_reduce, dim3((D + kThreads - 1) / kThreads), dim3(kThreads), 0, st, A, D);
      mark(K_NORM_REDUCE, 1);
    }
  }
  return hipGetLastError();
}

template <class T>
hipError_t dispatch(int D, const NormArgs& A, hipStream_t st, int backward) {
  switch (D) {
    case 16: return launch<16, T>(A, st, backward);
    case 32: return launch<32, T>(A, st, backward);
    case 64: return launch<64, T>(A, st, backward);
    case 128: return launch<128, T>(A, st, backward);
    case 256: return launch<256, T>(A, st, backward);
  }
  return hipErrorInvalidValue;
}

int validate(const tjev_gdn_norm_params* p) {
  if (!p) return fail(TJEV_GDN_EINVAL, "null params");
  if (p->tokens < 0 || p->heads <= 0) return fail(TJEV_GDN_EINVAL, "tokens must be >= 0 and heads > 0");
  if (p->dtype != TJEV_GDN_F32 && p->dtype != TJEV_GDN_BF16)
    return fail(TJEV_GDN_EINVAL, "dtype must be TJEV_GDN_F32 or TJEV_GDN_BF16");
  if (!(p->eps >= 0.f)) return fail(TJEV_GDN_EINVAL, "eps must be >= 0");
  const int d = p->dim;
  if (d != 16 && d != 32 && d != 64 && d != 128 && d != 256)
    return fail(TJEV_GDN_EUNSUPPORTED, "gated RMSNorm kernels exist for dim 16, 32, 64, 128 and 256");
  if (p->tokens * (long)p->heads * d > (1L << 40)) return fail(TJEV_GDN_EINVAL, "problem too large");
  return 0;
}

int bwd_blocks(const tjev_gdn_norm_params* p) {
  const long rpb = kThreads / (p->dim / 8);  // rows per workgroup iteration
  const long need = (p->tokens * p->heads + rpb - 1) / rpb;
  return (int)(need < kMaxBwdBlocks ? (need > 0 ? need : 1) : kMaxBwdBlocks);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

NormArgs base(const tjev_gdn_norm_params* p) {
  NormArgs A{};
  A.rows = p->tokens * p->heads;
  A.heads = p->heads;
  A.eps = p->eps;
  return A;
}

int run(const tjev_gdn_norm_params* p, const NormArgs& A, void* stream, int backward) {
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const hipError_t e = p->dtype == TJEV_GDN_BF16 ? dispatch<uint16_t>(p->dim, A, st, backward)
                                                 : dispatch<float>(p->dim, A, st, backward);
  if (e != hipSuccess) return fail(TJEV_GDN_EHIP, hipGetErrorString(e));
  return 0;
}

}  // namespace
}  // namespace gdn

extern "C" {

size_t tjev_gdn_norm_workspace_bytes(const tjev_gdn_norm_params* p, int weight_grad) {
  if (gdn::validate(p) || !weight_grad) return 0;
  return (size_t)gdn::bwd_blocks(p) * p->dim * sizeof(float);
}

int tjev_gdn_gated_rmsnorm_fwd(const tjev_gdn_norm_params* p, void* stream, const void* x, const void* gate,
                               const float* weight, const int32_t* seg, void* y) {
  if (int s = gdn::validate(p)) return s;
  if (p->tokens == 0) return 0;  // empty tensors may have null data pointers
  if (!x || !gate || !weight || !y) return gdn::fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (!gdn::aligned16(x) || !gdn::aligned16(gate) || !gdn::aligned16(y))
    return gdn::fail(TJEV_GDN_EINVAL, "x, gate and y must be 16-byte aligned");
  gdn::NormArgs A = gdn::base(p);
  A.x = x;
  A.z = gate;
  A.w = weight;
  A.seg = seg;
  A.y = y;
  return gdn::run(p, A, stream, 0);
}

int tjev_gdn_gated_rmsnorm_bwd(const tjev_gdn_norm_params* p, void* stream, const void* x, const void* gate,
                               const float* weight, const int32_t* seg, const void* d_y, void* d_x, void* d_gate,
                               float* d_weight, void* workspace, size_t workspace_bytes) {
  if (int s = gdn::validate(p)) return s;
  if (!weight || (p->tokens && (!x || !gate || !d_y || !d_x || !d_gate)))
    return gdn::fail(TJEV_GDN_EINVAL, "null tensor argument");
  if (!gdn::aligned16(x) || !gdn::aligned16(gate) || !gdn::aligned16(d_y) || !gdn::aligned16(d_x) ||
      !gdn::aligned16(d_gate))
    return gdn::fail(TJEV_GDN_EINVAL, "x, gate, d_y, d_x and d_gate must be 16-byte aligned");
  const size_t need = tjev_gdn_norm_workspace_bytes(p, d_weight != nullptr);
  if (need && (!workspace || workspace_bytes < need))
    return gdn::fail(TJEV_GDN_EWORKSPACE, "the weight gradient needs a workspace of tjev_gdn_norm_workspace_bytes");
  gdn::NormArgs A = gdn::base(p);
  A.x = x;
  A.z = gate;
  A.w = weight;
  A.seg = seg;
  A.dy = d_y;
  A.dx = d_x;
  A.dz = d_gate;
  // no rows: no backward launch, and the reduce writes d_weight = 0 from no partials
  A.nblk = p->tokens ? gdn::bwd_blocks(p) : 0;
  A.dwp = d_weight ? static_cast<float*>(workspace) : nullptr;
  A.dw = d_weight;
  return gdn::run(p, A, stream, 1);
}

}  // extern "C"
