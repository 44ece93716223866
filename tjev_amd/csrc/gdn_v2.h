// The v2 operator's ends (tjev's chunk_gated_delta_rule_v2, pallas_tpu_v2.py:541-582): the
// delta rule on given q, k [B,T,Hk,D], v [B,T,H,D], g, beta [B,T,H] -- no conv, no l2norm, no
// gate functions -- around the same chunk, scan and output kernels as the megakernel. q and k
// are taken as given (the model passes l2norm(q) * Dk^-1/2 and l2norm(k), gdn.py:90-92); the
// padded tail (t >= T) has zero inputs and the last token's segment id (xla.py:198-204; the
// segment-0 padding of pallas_tpu_v2.py:565-569 gives the same outputs).
#pragma once

#include "gdn_kernels.h"

namespace gdn {

// ---------------------------------------------------------------- k_prep_v2
// grid (B*N, 2*Hk + H), 256 threads: slot y copies q head y (< Hk), k head y - Hk or v head
// y - 2Hk of the chunk into the head-major fp32 workspace; the value heads also take the
// in-chunk cumulative g (fp64, kept as an fp32 high/low pair) and beta, and slot 0 writes
// the padded segment ids.
template <int C, int D, class TIO, class TQK, class TG>
__global__ __launch_bounds__(256) void k_prep_v2(GdnArgs A) {
  constexpr int CG = D / 8;
  constexpr int RPP = 256 / CG;
  const int b = blockIdx.x / A.N, n = blockIdx.x % A.N;
  const int slot = blockIdx.y;
  const int cg = threadIdx.x % CG;
  const int kind = slot < A.Hk ? 0 : (slot < 2 * A.Hk ? 1 : 2);
  const int head = kind == 0 ? slot : (kind == 1 ? slot - A.Hk : slot - 2 * A.Hk);
  const int heads = kind < 2 ? A.Hk : A.H;
  float* dst = kind == 0 ? A.qn + hoff(A, b, head, A.Hk, n, C, D)
             : kind == 1 ? A.kn + hoff(A, b, head, A.Hk, n, C, D)
                         : A.vv + hoff(A, b, head, A.H, n, C, D);
  for (int r = threadIdx.x / CG; r < C; r += RPP) {
    const int t = n * C + r;
    float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (t < A.T) {
      const size_t at = (((size_t)b * A.T + t) * heads + head) * D + cg * 8;
      if (kind < 2) {
        ld8(reinterpret_cast<const TQK*>(kind == 0 ? A.q2 : A.k2) + at, x);
      } else {
        ld8(reinterpret_cast<const TIO*>(A.v2) + at, x);
      }
    }
    float4* o = reinterpret_cast<float4*>(dst + (size_t)r * D + cg * 8);
    o[0] = make_float4(x[0], x[1], x[2], x[3]);
    o[1] = make_float4(x[4], x[5], x[6], x[7]);
  }
  if (slot == 0) {
    for (int i = threadIdx.x; i < C; i += 256) {
      const int t = n * C + i;
      A.segp[(size_t)b * A.Tp + t] = A.seg[(size_t)b * A.T + (t < A.T ? t : A.T - 1)];  // edge mode
    }
  }
  if (kind == 2 && threadIdx.x < 64) {  // gamma = in-chunk inclusive cumsum of g (fp64), beta
    constexpr int E = (C + 63) / 64;
    const int l = threadIdx.x;
    const TG* gg = reinterpret_cast<const TG*>(A.g2);
    const TG* gb = reinterpret_cast<const TG*>(A.b2);
    double g[E], run = 0.0;
    float bt[E];
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int i = l * E + q, t = n * C + i;
      const bool in = i < C && t < A.T;
      run += in ? (double)ldf(gg + ((size_t)b * A.T + t) * A.H + head) : 0.0;
      g[q] = run;
      bt[q] = in ? ldf(gb + ((size_t)b * A.T + t) * A.H + head) : 0.f;
    }
    double inc = run;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const double up = __shfl_up(inc, d);
      if (l >= d) inc += up;
    }
    const double excl = inc - run;
    const size_t tok = (size_t)(b * A.H + head) * A.Tp + (size_t)n * C;
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int i = l * E + q;
      if (i < C) {
        const double gm = excl + g[q];
        const float hi = (float)gm;
        A.gam[tok + i] = hi;
        A.gaml[tok + i] = (float)(gm - (double)hi);
        A.bet[tok + i] = bt[q];
      }
    }
  }
}

// ---------------------------------------------------------------- k_post_v2
// grid (B*N, 2*Hk + H), 256 threads: d q and d k per key head (the sum over its value heads,
// the GQA of pallas_tpu_v2's index maps), d v = X beta, d beta = rows(dkb, k) + rows(X, v),
// d g = the reverse in-chunk cumsum of d gamma (fp64).
template <int C, int D, class TIO, class TQK, class TG>
__global__ __launch_bounds__(256) void k_post_v2(GdnArgs A) {
  constexpr int CG = D / 8;
  constexpr int RPP = 256 / CG;
  __shared__ float sxv[C];
  const int b = blockIdx.x / A.N, n = blockIdx.x % A.N;
  const int slot = blockIdx.y;
  const int cg = threadIdx.x % CG;
  const int kind = slot < A.Hk ? 0 : (slot < 2 * A.Hk ? 1 : 2);
  const int head = kind == 0 ? slot : (kind == 1 ? slot - A.Hk : slot - 2 * A.Hk);
  for (int r = threadIdx.x / CG; r < C; r += RPP) {
    const int t = n * C + r;
    if (kind < 2) {
      if (t >= A.T) continue;
      const float* src = (kind == 0 ? A.dqh : A.dkh) + ((size_t)(b * A.H + head * A.ratio) * A.Tp + t) * D + cg * 8;
      float d[8];
      ld8(src, d);
      for (int v = 1; v < A.ratio; ++v) {
        float y[8];
        ld8(src + (size_t)v * A.Tp * D, y);
#pragma unroll
        for (int e = 0; e < 8; ++e) d[e] += y[e];
      }
      st8_io(reinterpret_cast<TQK*>(kind == 0 ? A.d_q2 : A.d_k2) + (((size_t)b * A.T + t) * A.Hk + head) * D + cg * 8, d);
    } else {
      const size_t row = ((size_t)(b * A.H + head) * A.Tp + t) * D + cg * 8;
      float x[8], v[8];
      ld8(A.xl + row, x);
      ld8(A.vv + row, v);
      const float bt = A.bet[(size_t)(b * A.H + head) * A.Tp + t];
      float xv = 0.f, d[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        d[e] = x[e] * bt;
        xv += x[e] * v[e];
      }
      xv = sum_lanes<CG>(xv);
      if (cg == 0) sxv[r] = xv;
      if (t < A.T) st8_io(reinterpret_cast<TIO*>(A.d_v2) + (((size_t)b * A.T + t) * A.H + head) * D + cg * 8, d);
    }
  }
  __syncthreads();
  if (kind == 2 && threadIdx.x < 64) {
    constexpr int E = (C + 63) / 64;
    const int l = threadIdx.x;
    TG* dg = reinterpret_cast<TG*>(A.d_g2);
    TG* db = reinterpret_cast<TG*>(A.d_b2);
    const size_t tok = (size_t)(b * A.H + head) * A.Tp + (size_t)n * C;
    float ta[E], tf[E], tx[E];
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int ic = l * E + q < C ? l * E + q : C - 1;
      ta[q] = A.dgam[tok + ic];
      tf[q] = A.dkws[tok + ic];
      tx[q] = A.dcross[tok + ic];
    }
    double dgv[E];
    chunk_dg<C, E>(ta, tf, tx, dgv);
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int i = l * E + q, t = n * C + i;
      if (i < C && t < A.T) {
        stf(dg + ((size_t)b * A.T + t) * A.H + head, (float)dgv[q]);
        stf(db + ((size_t)b * A.T + t) * A.H + head, A.dbet[tok + i] + sxv[i]);
      }
    }
  }
}

}  // namespace gdn
