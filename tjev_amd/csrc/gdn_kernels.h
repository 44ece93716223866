// The GDN megakernel's HIP kernels for gfx950, as templates over the chunk C, the head dim
// D (= Dk = Dv), the arithmetic of the intra-chunk products PI and of the state-path
// products PS, and the storage type of the activations (float or bf16 as uint16_t).
//
// Forward (reference: pallas_tpu_mega.py:216-249 with pallas_tpu_v2.py:212-269):
//   k_prep      conv + SiLU + padding mask, l2norm(q, k), q * Dk^-1/2, gates beta, g and the
//               in-chunk cumulative decay gamma; head-major fp32 tiles      (HBM-bound)
//   k_chunk     per (row, head, chunk): L = strict(beta k k^T . D), T = (I+L)^-1 (16x16
//               diagonal blocks by doubling or by substitution, then doubling levels on
//               MFMA), w = T kbe, u = T v beta                                (MFMA)
//   k_scan_fwd  per (row, head, Dv tile): the recurrent state S (Dk x Dv tile, fp32), chunks
//               in order: S_before stored, v_new = u - w S, S = carry S + k_write^T v_new
//   k_out       per chunk: o = q_read S_before + ((q k^T) . D) v_new        (MFMA)
// Backward (reference: pallas_tpu_mega.py:252-319 with pallas_tpu_v2.py:272-318):
//   k_prep (recomputed), k_chunk (mode 1: T kept, v_new = u - w S_before recomputed from the
//   saved chunk-boundary states), k_bwd_local (X_loc = T^T intra^T do, Kt = T^T k_write),
//   k_scan_bwd (chunks reversed: X = X_loc + Kt G, G = carry G + q_read^T do - kbe^T X),
//   k_bwd_grads (dq, dk per value head, d gamma, d beta), k_post (GQA sums, l2norm, SiLU and
//   conv backward, gate backward), k_reduce (d A_log, d dt_bias, d conv weight).
#pragma once

#include "gdn_args.h"
#include "gdn_device.h"

namespace gdn {

// Storage of the chunk-boundary states (the residual S): bf16 when the state-path products are one
// bf16 pass (precisions mixed and bf16), else fp32, as the reference keeps them
// (pallas_tpu_mega.py:425-426, _state_dtypes). Every reader of S in those modes feeds it to a
// one-pass bf16 product, which rounds it to bf16 anyway, except the carry's gradient
// <G_after, S_before> (the reference reads its bf16 S there too) and the final state, which
// k_final_state builds from an fp32 copy of the last chunk's S (GdnArgs::s_last).
template <int PS>
using StateT = std::conditional_t<PS == P_BF16, uint16_t, float>;
template <int PS>
__device__ __forceinline__ StateT<PS>* states_ptr(const GdnArgs& A) {
  return static_cast<StateT<PS>*>(A.states);
}
// Storage of T = (I + L)^-1 between kernels and as a residual: bf16 when the intra-chunk products
// are one bf16 pass (precision bf16, the reference's t_dtype), else fp32. T only ever enters
// those products.
template <int PI>
using TinvT = std::conditional_t<PI == P_BF16, uint16_t, float>;
template <int PI>
__device__ __forceinline__ TinvT<PI>* tinv_ptr(const GdnArgs& A) {
  return static_cast<TinvT<PI>*>(A.tt);
}

__device__ __forceinline__ size_t hoff(const GdnArgs& A, int b, int head, int heads, int n, int C, int D) {
  return ((size_t)(b * heads + head) * A.Tp + (size_t)n * C) * D;
}

// g + row * ld + col for a lane's element of a staged tile (all three small) from a wave-uniform
// base g: with GDN_LANE_OFF32 as a 32-bit offset, so the loads take the scalar-base form (one
// VGPR per address instead of a 64-bit pair), else widened before the multiply. Which form
// allocates better is a property of the kernel (a spilled address reloaded from scratch waits
// for every outstanding memory operation), so each object file of gdn_inst.hip sets it for its
// kernel family.
#ifndef GDN_LANE_OFF32
#define GDN_LANE_OFF32 0
#endif
template <class T>
__device__ __forceinline__ const T* lane_ptr(const T* g, int row, int ld, int col) {
  if constexpr (GDN_LANE_OFF32) {
    return g + (unsigned)(row * ld + col);
  } else {
    return g + (size_t)row * ld + col;
  }
}

// ---------------------------------------------------------------- chunk context
// Segment semantics (pallas_tpu_v2.py:226-241, pallas_tpu_mega.py:349-361): cont_i: token i
// reads the incoming state (same id as the previous chunk's last token; before chunk 0: -2, or
// token 0's id when the sequence continues from an initial state, xla.py:214-216); in_last_i:
// token i writes the outgoing state (same id as the chunk's last token).
template <int C>
struct Ctx {
  int seg[C];
  float gam[C], gaml[C], beta[C], grow[C], kws[C], bg[C];
  int before;
  int hseg[3];  // ids of tokens nC - 1, nC - 2, nC - 3 (token 0's in chunk 0), with CtxRaw's HALO
  float carry;
};

// gamma_i - gamma_j from the (high, low) pairs: the high parts of nearby tokens subtract
// exactly, so the decays keep the accuracy of the fp64 prefix sum
template <int C>
__device__ __forceinline__ float gdiff(const Ctx<C>& cx, int i, int j) {
  return (cx.gam[i] - cx.gam[j]) + (cx.gaml[i] - cx.gaml[j]);
}

// dg_t = sum_{s >= t} a_s + sum_{s < t} f_s + x_t over one chunk's tokens, in fp64 (the
// gradient of the log decays from k_bwd_grads' three per-token terms). One wave; lane l holds
// tokens l E .. l E + E - 1 (values of tokens past the chunk are ignored).
template <int C, int E>
__device__ __forceinline__ void chunk_dg(const float (&a)[E], const float (&f)[E], const float (&x)[E],
                                         double (&dg)[E]) {
  const int l = lane();
  double sa[E], pf[E], run = 0.0, runf = 0.0;
#pragma unroll
  for (int q = E - 1; q >= 0; --q) {  // inclusive suffix of a within the lane
    run += l * E + q < C ? (double)a[q] : 0.0;
    sa[q] = run;
  }
#pragma unroll
  for (int q = 0; q < E; ++q) {  // exclusive prefix of f within the lane
    pf[q] = runf;
    runf += l * E + q < C ? (double)f[q] : 0.0;
  }
  double inc = run, incf = runf;  // across the lanes: a suffix scan of a, a prefix scan of f
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const double dn = __shfl_down(inc, d);
    const double up = __shfl_up(incf, d);
    if (l + d < 64) inc += dn;
    if (l >= d) incf += up;
  }
  const double ea = inc - run, ef = incf - runf;
#pragma unroll
  for (int q = 0; q < E; ++q) dg[q] = ea + sa[q] + ef + pf[q] + (double)x[q];
}

// One 16 x 16 tile of E (rows i of the wave's strip at acc_row(rr), columns j = 16 t +
// acc_col()) into the sums over token pairs across t, x_t = sum_{i >= t > j} E_ij: rp[rr] holds
// row i's sum over the columns before the tile and is advanced past it; cp gets, for the lane's
// column t, the sum over the strip's rows i >= t of row i's sum over j < t (diag: the tile on
// the strip's diagonal, where only rows i >= t count; E is zero for j >= i). The prefixes along
// a row are DPP shifts within the lane's 16-lane row.
__device__ __forceinline__ void cross_tile(const f32x4& e, bool diag, float (&rp)[4], float& cp) {
  const int c = acc_col();
  float col = 0.f;
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    float inc = e[rr];  // inclusive prefix over the tile's 16 columns (row_shr 1, 2, 4, 8)
    inc += dpp_read<0x111>(inc);
    inc += dpp_read<0x112>(inc);
    inc += dpp_read<0x114>(inc);
    inc += dpp_read<0x118>(inc);
    const float pre = rp[rr] + dpp_read<0x111>(inc);  // exclusive: 0 in the row's first lane
    col += (!diag || acc_row(rr) >= c) ? pre : 0.f;
    rp[rr] += sum16(e[rr]);
  }
  col += __shfl_xor(col, 16);
  col += __shfl_xor(col, 32);
  cp += col;
}

// The per-token inputs of one chunk's context held in registers (thread i < C holds token i):
// fetch() issues the loads, commit() writes them to the LDS context (derive_ctx then fills in
// the rest). Needs at least C threads.
template <int C, bool HALO = false>
struct CtxRaw {
  int seg, before;
  float gam, gaml, beta;
  bool first;  // chunk 0: the token before it is "-2", or token 0's id (loaded) with an initial state
  // Every thread loads (threads past C repeat token threadIdx.x % C), with no branch around the
  // loads: a fixed count of memory operations per wave lets the compiler wait for exactly the
  // loads it needs instead of for all outstanding ones.
  __device__ __forceinline__ void fetch(const GdnArgs& A, int b, int h, int n) {
    const int i = threadIdx.x % C;
    const size_t tok = (size_t)(b * A.H + h) * A.Tp + (size_t)n * C + i;
    seg = A.segp[(size_t)b * A.Tp + (size_t)n * C + i];
    gam = A.gam[tok];
    gaml = A.gaml[tok];
    beta = A.bet[tok];
    // HALO: threads 1 and 2 (and their repeats) load the ids of the two tokens before that one
    before = A.segp[(size_t)b * A.Tp + (n > 0 ? (size_t)n * C - 1 - (HALO ? (i < 2 ? i : 2) : 0) : 0)];
    first = n == 0 && !A.init_state;
  }
  __device__ __forceinline__ void commit(Ctx<C>& cx) const {
    const int i = threadIdx.x;
    if (i < C) {
      cx.seg[i] = seg;
      cx.gam[i] = gam;
      cx.gaml[i] = gaml;
      cx.beta[i] = beta;
    }
    if (i == 0) cx.before = first ? -2 : before;
    if (HALO && i < 3) cx.hseg[i] = before;
  }
};

template <int C, int NT>
__device__ __forceinline__ void derive_ctx(Ctx<C>& cx);

template <int C, int NT>
__device__ __forceinline__ void load_ctx(Ctx<C>& cx, const GdnArgs& A, int b, int h, int n) {
  static_assert(NT >= C, "one thread per token");
  CtxRaw<C> raw;
  raw.fetch(A, b, h, n);
  raw.commit(cx);
  __syncthreads();
  derive_ctx<C, NT>(cx);
  __syncthreads();
}

// grow, kws, bg and carry from seg, gamma and beta (the LDS context written, then synced)
template <int C, int NT>
__device__ __forceinline__ void derive_ctx(Ctx<C>& cx) {
  for (int i = threadIdx.x; i < C; i += NT) {
    const bool cont = cx.seg[i] == cx.before;
    const bool in_last = cx.seg[i] == cx.seg[C - 1];
    cx.grow[i] = cont ? expf(cx.gam[i] + cx.gaml[i]) : 0.f;        // e^gamma . cont
    cx.kws[i] = in_last ? expf(gdiff(cx, C - 1, i)) : 0.f;          // e^(gamma_C - gamma) . in_last
    cx.bg[i] = cx.beta[i] * cx.grow[i];                              // kbe = k . beta . grow
  }
  if (threadIdx.x == 0) cx.carry = (cx.seg[C - 1] == cx.before) ? expf(cx.gam[C - 1] + cx.gaml[C - 1]) : 0.f;
}

// D_ij = e^(gamma_i - gamma_j) on same-segment i >= j, else 0, over one wave's 16-row strip
// (rows i0 + acc_row(rr)), tile by tile. Below the diagonal the exponential factors through
// the strip's first row p = i0: for j < p <= i,
// e^(gamma_i - gamma_j) = e^(gamma_i - gamma_p) e^(gamma_p - gamma_j) with both factors <= 1
// (gamma never increases along a chunk: g <= 0), so a lane takes 4 exponentials for its rows
// and 1 per tile instead of 4 per tile; the diagonal tile takes each one directly.
template <int C>
struct StripDecay {
  float a[4];  // e^(gamma_i - gamma_p) of the lane's rows
  int s[4];    // their segment ids
  __device__ __forceinline__ StripDecay(const Ctx<C>& cx, int i0) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int i = i0 + acc_row(rr);
      a[rr] = expf(gdiff(cx, i, i0));
      s[rr] = cx.seg[i];
    }
  }
  // d[rr] = D(i0 + acc_row(rr), 16t + acc_col()) for the strip of wave w (i0 = 16w)
  __device__ __forceinline__ void tile(const Ctx<C>& cx, int i0, int t, int w, float (&d)[4]) const {
    const int j = 16 * t + acc_col();
    const int sj = cx.seg[j];
    if (t < w) {
      const float b = expf(gdiff(cx, i0, j));
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) d[rr] = s[rr] == sj ? a[rr] * b : 0.f;
    } else if (t == w) {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = i0 + acc_row(rr);
        d[rr] = (i >= j && s[rr] == sj) ? expf(gdiff(cx, i, j)) : 0.f;
      }
    } else {
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) d[rr] = 0.f;
    }
  }
};

// R x D fp32 tile from global (row stride D) into LDS (row stride LD), every load issued first
template <int R, int D, int NT, class TS>
__device__ __forceinline__ void load_tile(float* s, int LD, const TS* g);

// The order in which a persistent kernel walks its units (workgroup i takes units i, i + grid,
// ...). A kernel's last units are still in the L2 and memory-side caches when the next kernel
// starts, so a producer whose consumer is a scan ends on the chunks the scan reads first:
//   BY_HEAD      all chunks of a (row, head) together
//   CHUNKS_DOWN  one chunk of every (row, head) at a time, the last chunk first (k_chunk: the
//                forward scan and k_bwd_local start from chunk 0)
//   CHUNKS_UP    the same, chunk 0 first (k_bwd_local: the backward scan starts from the last)
enum UnitOrder { BY_HEAD, CHUNKS_DOWN, CHUNKS_UP };

// indices of the (row, head, chunk) unit u of the chunk-parallel kernels
template <UnitOrder O>
struct UnitIx {
  int n, bh, h, b, hk;
  __device__ __forceinline__ UnitIx(const GdnArgs& A, int u) {
    if constexpr (O == BY_HEAD) {
      n = u % A.N;
      bh = u / A.N;
    } else {
      const int nbh = A.B * A.H, c = u / nbh;
      bh = u - c * nbh;
      n = O == CHUNKS_DOWN ? A.N - 1 - c : c;
    }
    h = bh % A.H;
    b = bh / A.H;
    hk = h / A.ratio;
  }
};

// ---------------------------------------------------------------- inverse
// (I + L)^-1 in place for the strictly lower-triangular L in sT (C x C, row stride LT): the
// 16x16 diagonal blocks first (one wave per block), then doubling levels s = 16 .. C/2 on
// MFMA, T_LL = -T_BR (L_LL T_TL) (pallas_tpu_v2.py:144-193; xla.py:82-100). The diagonal
// blocks either by the doubling levels s = 1, 2, 4, 8 from T = I at the products' precision
// (inverse "doubling": the whole inverse is the pure doubling) or exactly by forward
// substitution on the VALU (inverse "blocked"). sTT (C x LT floats) keeps T transposed as it is built, so the right
// operand T_TL is read by rows. A level's product L_LL T_TL is kept transposed in the pair's
// upper-right block of sT (unused by a lower-triangular T) and read by rows in turn. Products
// with a triangular operand run over whole 32-wide contraction steps, so they read the upper
// 16 x 16 corners of the 32 x 32 diagonal blocks of sT (and the lower corners of sTT): those
// hold zeros when read (the level-16 products kept there are cleared at level 32, or at the
// end when C = 32). On return sT holds T with the upper triangle zero wherever a product with
// 32-wide steps reads it, and the level products elsewhere above the diagonal; the caller
// synchronises before reading sT.
template <int C, int P, int S>
__device__ __forceinline__ void doubling_level(float* sT, float* sTT, int LT) {
  if constexpr (S < C) {
    constexpr int TPS = S / 16;                 // 16-wide tiles per side of a pair's block
    constexpr int TW = S >= 32 ? S / 32 : 1;    // tiles per wave, all in one row strip
    const int w = wave(), l = lane();
    const int strip = w >> 1, half = w & 1;     // C/32 row strips of 16 rows, two waves each
    const int p = strip / TPS, ti = strip % TPS;
    const int r0 = 2 * S * p;
    const int tj0 = half * TW;
    const bool on = S >= 32 || half == 0;
    const int c = acc_col(), g4 = (l >> 4) << 2;
    if (on) {  // tmp = L_LL T_TL for rows 16 ti, kept transposed at sT[r0 + j][r0 + S + i]
      f32x4 acc[TW];
      zero(acc);
      strip_mma<P, S, TW>(acc, krow(sT + (r0 + S) * LT + r0, LT), 16 * ti, krow(sTT + r0 * LT + r0, LT), 16 * tj0,
                          tri_begin(16 * tj0));
#pragma unroll
      for (int t = 0; t < TW; ++t)
        *reinterpret_cast<float4*>(sT + (r0 + 16 * (tj0 + t) + c) * LT + r0 + S + 16 * ti + g4) =
            make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    }
    if constexpr (S == 32) {  // clear the level-16 products: read as zeros from the next phase on
      for (int idx = threadIdx.x; idx < (C / 32) * 256; idx += C * 4) {
        const int q = idx >> 8, r = (idx >> 4) & 15, k = idx & 15;
        sT[(32 * q + r) * LT + 32 * q + 16 + k] = 0.f;
      }
    }
    __syncthreads();
    if (on) {  // T_LL = -T_BR tmp
      f32x4 acc[TW];
      zero(acc);
      strip_mma<P, S, TW>(acc, krow(sT + (r0 + S) * LT + r0 + S, LT), 16 * ti, krow(sT + r0 * LT + r0 + S, LT),
                          16 * tj0, 0, tri_end<S>(16 * ti));
#pragma unroll
      for (int t = 0; t < TW; ++t) {
        const int j = r0 + 16 * (tj0 + t) + c, i = r0 + S + 16 * ti + g4;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) lds_st(sT + (i + rr) * LT + j, -acc[t][rr]);
        if constexpr (2 * S < C)  // the last level's T_TL is never read again
          *reinterpret_cast<float4*>(sTT + j * LT + i) = make_float4(-acc[t][0], -acc[t][1], -acc[t][2], -acc[t][3]);
      }
    }
    __syncthreads();
    doubling_level<C, P, 2 * S>(sT, sTT, LT);
  }
}

// One 16 x 16 x 16 product at precision P of tiles held at the accumulator layout (lane l: rows
// 4 (l / 16) + e, column l % 16): a[e] = A(l % 16, 4 (l / 16) + e), b[e] = B(4 (l / 16) + e, l % 16).
// A tile X at that layout is thus both the B operand X and the A operand X^T. The contraction's
// 16 values fill the first four of each lane group's eight slots of a 32-deep step; the rest
// are zero.
template <int P>
__device__ __forceinline__ f32x4 mma16(const float (&a)[4], const float (&b)[4]) {
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (P == P_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  } else {
    const float xa[8] = {a[0], a[1], a[2], a[3], 0.f, 0.f, 0.f, 0.f};
    const float xb[8] = {b[0], b[1], b[2], b[3], 0.f, 0.f, 0.f, 0.f};
    mma<P>(acc, make_frag<a_prec<P>()>(xa), make_frag<b_prec<P>()>(xb));
  }
  return acc;
}

// (I + L_d)^-1 of one 16 x 16 diagonal block by the doubling levels s = 1, 2, 4, 8 from T = I
// (xla.py:82-100, pallas_tpu_v2.py:168-193): T <- T - (T off) T, off the lower-left s x s block
// of every 2s x 2s block of L, each product at precision P and rounded to fp32 as the
// reference's. lo, t and tt at the accumulator layout (L, T and T^T): P^T = off^T T^T, then
// Q = P T and Q^T = T^T P^T, every operand already in registers.
template <int P>
__device__ __forceinline__ void diag_doubling(const float (&lo)[4], float (&t)[4], float (&tt)[4]) {
  const int j = lane() & 15, i0 = (lane() >> 4) << 2;
#pragma unroll
  for (int r = 0; r < 4; ++r) t[r] = tt[r] = i0 + r == j ? 1.f : 0.f;
#pragma unroll
  for (int lv = 0; lv < 4; ++lv) {
    float off[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int i = i0 + r;
      const bool m = (i >> (lv + 1)) == (j >> (lv + 1)) && ((i >> lv) & 1) && !((j >> lv) & 1);
      off[r] = m ? lo[r] : 0.f;
    }
    const f32x4 pv = mma16<P>(off, tt);
    const float pt[4] = {pv[0], pv[1], pv[2], pv[3]};
    const f32x4 q = mma16<P>(pt, t);
    const f32x4 qt = mma16<P>(t, pt);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      t[r] -= q[r];
      tt[r] -= qt[r];
    }
  }
}

template <int C, int P>
__device__ __forceinline__ void invert_unit_lower(float* sT, int LT, float* sTT, bool doubling) {
  const int w = wave(), l = lane();
  if (doubling) {  // the wave's diagonal block in registers; sT and sTT get T and T^T
    const int j = l & 15, i0 = (l >> 4) << 2;
    float* blk = sT + 16 * w * LT + 16 * w;
    float* blkT = sTT + 16 * w * LT + 16 * w;
    float lo[4], t[4], tt[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) lo[r] = blk[(i0 + r) * LT + j];
    diag_doubling<P>(lo, t, tt);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      lds_st(blk + (i0 + r) * LT + j, t[r]);
      lds_st(blkT + (i0 + r) * LT + j, tt[r]);
    }
    if (w % 2 == 1) {  // zeros in sTT's lower 16 x 16 corner of the 32 x 32 diagonal block
      for (int idx = l; idx < 256; idx += 64) {
        const int r = idx >> 4, k = idx & 15;
        sTT[(16 * w + r) * LT + 16 * (w - 1) + k] = 0.f;
      }
    }
  } else if (l < 16) {  // diagonal block w: lane l owns column l, X[i] = e_i - sum_{r<i} L[i][r] X[r]
    const float* blk = sT + 16 * w * LT + 16 * w;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (i == l) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      float row[16];
#pragma unroll
      for (int q = 0; q < (i + 3) / 4; ++q) {  // L[i][0 .. i-1], the same words for every lane
        const float4 v = *reinterpret_cast<const float4*>(blk + i * LT + 4 * q);
        row[4 * q] = v.x;
        row[4 * q + 1] = v.y;
        row[4 * q + 2] = v.z;
        row[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int r = 0; r < i; ++r) x[i] -= row[r] * x[r];
    }
    float* out = sT + 16 * w * LT + 16 * w + l;
#pragma unroll
    for (int i = 0; i < 16; ++i) lds_st(out + i * LT, x[i]);
    float4* outT = reinterpret_cast<float4*>(sTT + (16 * w + l) * LT + 16 * w);
#pragma unroll
    for (int q = 0; q < 4; ++q) outT[q] = make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
  } else if (w % 2 == 1) {  // zeros in sTT's lower 16 x 16 corner of the 32 x 32 diagonal block
    for (int idx = l - 16; idx < 256; idx += 48) {
      const int r = idx >> 4, k = idx & 15;
      sTT[(16 * w + r) * LT + 16 * (w - 1) + k] = 0.f;
    }
  }
  __syncthreads();
  doubling_level<C, P, 16>(sT, sTT, LT);
  if constexpr (C == 32) {  // no level 32 to clear the level-16 product
    for (int idx = threadIdx.x; idx < 256; idx += C * 4) sT[(idx >> 4) * LT + 16 + (idx & 15)] = 0.f;
  }
}

// ---------------------------------------------------------------- conv helpers
// Per-lag conv weights of 8 channels: wl[L] multiplies token t-L (w[K-1-L]), zero past the taps.
// Static lag indices keep them in registers.
__device__ __forceinline__ void lag_weights(const GdnArgs& A, int cc, float (&wl)[5][8]) {
#pragma unroll
  for (int L = 0; L < 5; ++L)
#pragma unroll
    for (int e = 0; e < 8; ++e) wl[L][e] = (L < A.taps) ? A.conv_w[(size_t)(A.taps - 1 - L) * A.W + cc + e] : 0.f;
}

// Raw row tt (>= -(taps - 1)) of batch row b at channels cc..cc+7: rows before the row come
// from the conv history of a continued sequence (A.init_conv, oldest first), or read row 0 (a
// clamped address; the conv's tap masks drop them); rows past T read row T - 1 (padding).
template <class TIO>
__device__ __forceinline__ const TIO* halo_row(const GdnArgs& A, const TIO* x, int b, int tt, int cc) {
  const int k1 = A.taps > 0 ? A.taps - 1 : 0;
  const TIO* hist = reinterpret_cast<const TIO*>(A.init_conv);
  if (tt < 0 && hist && tt >= -k1) return hist + ((size_t)b * k1 + (k1 + tt)) * A.W + cc;
  return x + ((size_t)b * A.T + (tt < 0 ? 0 : (tt < A.T ? tt : A.T - 1))) * A.W + cc;
}

// ---------------------------------------------------------------- k_prep
// grid B*N*(2*Hk + H), 256 threads, the slot fastest: the workgroups of one chunk run together
// and read its token rows whole. Slot y: q head y (< Hk), k head y - Hk, v head y - 2Hk.
// Every (token, 8 channels) is independent: D/8 lanes per token row. l2norm of xla.py:42-53.
// Slot 0 first writes the padded segment ids of the chunk (read by every later kernel). With
// fuse_v the v slots only compute the gates (k_chunk builds the v rows from the raw ones), with
// fuse_q the q slots write nothing but slot 0's ids (k_out builds the q rows).
template <int C, int D, class TIO, class TG, int K1 = 4>
__global__ __launch_bounds__(256) void k_prep(GdnArgs A) {
  static_assert(K1 >= 1 && K1 <= 4, "conv lags 1..K1 (launched with K1 >= taps - 1)");
  constexpr int CG = D / 8;
  constexpr int RPP = 256 / CG;
  const int slots = 2 * A.Hk + A.H, bn = blockIdx.x / slots;
  const int b = bn / A.N, n = bn % A.N;
  const int slot = blockIdx.x % slots;
  const int cg = threadIdx.x % CG;
  int kind, head, c0;
  if (slot < A.Hk) { kind = 0; head = slot; c0 = slot * D; }
  else if (slot < 2 * A.Hk) { kind = 1; head = slot - A.Hk; c0 = A.Hk * D + head * D; }
  else { kind = 2; head = slot - 2 * A.Hk; c0 = 2 * A.Hk * D + head * D; }
  const int cc = c0 + cg * 8;
  const TIO* x = reinterpret_cast<const TIO*>(A.qkv);
  const int32_t* sg = A.seg + (size_t)b * A.T;
  float* dst = kind == 0 ? A.qn + hoff(A, b, head, A.Hk, n, C, D)
             : kind == 1 ? A.kn + hoff(A, b, head, A.Hk, n, C, D)
                         : A.vv + hoff(A, b, head, A.H, n, C, D);
  float wl[5][8];
  lag_weights(A, cc, wl);
  // Each group of CG lanes owns RG consecutive rows of the chunk and loads them with the HW rows
  // before them (the conv halo) and their segment ids at once, at clamped addresses without
  // branches; the conv then slides over registers (every raw row is read once).
  constexpr int RG = C / RPP > 0 ? C / RPP : 1;
  constexpr int HW = 4;  // taps - 1 <= 4 (a halo of 3 for taps <= 4 measured slower here)
  const int r0 = (threadIdx.x / CG) * RG;
  if ((RG * RPP == C || r0 < C) && !(kind == 2 && A.fuse_v) && !(kind == 0 && A.fuse_q)) {
    Raw8<TIO> raw[RG + HW];
    int sgv[RG + HW];
#pragma unroll
    for (int i = HW - K1; i < RG + HW; ++i) {  // the rows of lags past K1 are not read
      const int tt = n * C + r0 - HW + i;
      raw[i].load(halo_row<TIO>(A, x, b, tt, cc));
      sgv[i] = sg[tt < 0 ? 0 : (tt < A.T ? tt : A.T - 1)];  // rows before the row: token 0's segment
    }
    // every raw row converted to fp32 once (each is read by up to K1 + 1 rows' conv)
    float xr[RG + HW][8];
#pragma unroll
    for (int i = HW - K1; i < RG + HW; ++i) raw[i].get(xr[i]);
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      const int r = r0 + i, t = n * C + r;
      const int st = t < A.T ? sgv[HW + i] : 0;  // the padded tail: no activation
      float act[8];
      if (A.taps == 0) {  // mega1: qkv is already the activation (zero on the tail)
#pragma unroll
        for (int e = 0; e < 8; ++e) act[e] = t < A.T ? xr[HW + i][e] : 0.f;
      } else {  // z = sum over lags of keep * x[t-L] * w[K-1-L], lag 0 first (causal_conv1d.py:42-45)
        float z[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) z[e] = xr[HW + i][e] * wl[0][e];
#pragma unroll
        for (int L = 1; L <= K1; ++L) {
          const bool keep = L < A.taps && (t - L >= 0 || A.init_conv) && sgv[HW + i - L] == st;
#pragma unroll
          for (int e = 0; e < 8; ++e) z[e] = keep ? z[e] + xr[HW + i - L][e] * wl[L][e] : z[e];
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) act[e] = st > 0 ? z[e] * sigmoid_io<TIO>(z[e]) : 0.f;
      }
      if (kind < 2) {  // l2norm over the head's D channels (CG lanes)
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sq += act[e] * act[e];
        sq = sum_lanes<CG>(sq);
        float rn = sq == 0.f ? 0.f : 1.0f / sqrtf(sq + 1e-6f);
        if (kind == 0) rn *= A.scale;
#pragma unroll
        for (int e = 0; e < 8; ++e) act[e] *= rn;
      }
      float4* o = reinterpret_cast<float4*>(dst + (size_t)r * D + cg * 8);
      o[0] = make_float4(act[0], act[1], act[2], act[3]);
      o[1] = make_float4(act[4], act[5], act[6], act[7]);
    }
  }
  if (slot == 0) {  // the padded tail takes the last token's id (edge mode, xla.py:198-204)
    for (int i = threadIdx.x; i < C; i += 256) {
      const int t = n * C + i;
      A.segp[(size_t)b * A.Tp + t] = sg[t < A.T ? t : A.T - 1];
    }
  }
  if (kind == 2 && threadIdx.x < 64) {  // gates of value head `head` (pallas_tpu_mega.py:106-127)
    constexpr int E = (C + 63) / 64;
    const int l = threadIdx.x;
    const TG* ga = reinterpret_cast<const TG*>(A.ga);
    const TG* gb = reinterpret_cast<const TG*>(A.gb);
    const float alog = expf(A.a_log[head]), dtb = A.dt_bias[head];
    // gamma = in-chunk inclusive prefix sum of g, accumulated in fp64 and kept as fp32 hi + lo
    double g[E], run = 0.0;
    float bt[E];
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int i = l * E + q, t = n * C + i;
      const bool in = i < C && t < A.T;
      const float av = in ? ldf(ga + ((size_t)b * A.T + t) * A.H + head) : 0.f;
      const float bv = in ? ldf(gb + ((size_t)b * A.T + t) * A.H + head) : 0.f;
      run += in ? (double)(-alog * softplusf_(av + dtb)) : 0.0;  // the padded tail: g = 0, beta = 0
      g[q] = run;  // inclusive within the lane
      bt[q] = in ? sigmoidf_(bv) : 0.f;
    }
    double inc = run;  // inclusive scan of lane totals
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

// ---------------------------------------------------------------- operand staging
// An R x K fp32 tile held in registers, 4 consecutive values per slot: fetch() issues every
// global load of the tile at once (one memory round trip), the put_* calls then write it to an
// operand tile as stored (rows) or transposed (cols), scaled.
template <int R, int K, int NT, class TS = float>
struct Regs {
  static constexpr int V = K / 4;
  static constexpr int IT = (R * V + NT - 1) / NT;
  Packed4<TS> v[IT];  // as stored (fp32, or bf16 expanded when put)
  __device__ __forceinline__ static bool live(int it) {
    return (R * V) % NT == 0 || (int)threadIdx.x + it * NT < R * V;
  }
  __device__ __forceinline__ void fetch(const TS* g, int ldg) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int idx = threadIdx.x + it * NT;
      if (live(it)) v[it] = *reinterpret_cast<const Packed4<TS>*>(lane_ptr(g, idx / V, ldg, 4 * (idx % V)));
    }
  }
  // a lower triangular tile: only the 16 x 16 tiles on and below the diagonal are read. The
  // slots above go to the row's first tile (a line the same instruction fetches anyway), so
  // every slot still issues one load and the count stays static; put_lds_lower writes them as
  // zeros (the condition recomputed there, not held across the loads' latency).
  __device__ __forceinline__ static bool upper(int it) {
    const int idx = threadIdx.x + it * NT;
    return ((idx % V) >> 2) > ((idx / V) >> 4);
  }
  __device__ __forceinline__ void fetch_lower(const TS* g, int ldg) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int idx = threadIdx.x + it * NT, c4 = idx % V;
      if (live(it))
        v[it] = *reinterpret_cast<const Packed4<TS>*>(lane_ptr(g, idx / V, ldg, 4 * (upper(it) ? (c4 & 3) : c4)));
    }
  }
  __device__ __forceinline__ void put_lds_lower(float* s, int ld) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (!live(it)) continue;
      const int idx = threadIdx.x + it * NT;
      if constexpr (sizeof(TS) == 2) {
        *reinterpret_cast<float4*>(s + (idx / V) * ld + 4 * (idx % V)) =
            upper(it) ? make_float4(0.f, 0.f, 0.f, 0.f) : f4_of(v[it]);
      } else {
        *reinterpret_cast<float4*>(s + (idx / V) * ld + 4 * (idx % V)) = upper(it) ? make_float4(0.f, 0.f, 0.f, 0.f) : v[it];
      }
    }
  }
  // op(r, k) = g[r][k] * rs[r] * cst
  template <int P>
  __device__ __forceinline__ void put_rows(const Op<P>& op, const float* rs = nullptr, float cst = 1.f) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (!live(it)) continue;
      const int idx = threadIdx.x + it * NT, r = idx / V, c = 4 * (idx % V);
      const float f = (rs ? rs[r] : 1.f) * cst;
      if constexpr (sizeof(TS) == 2) {
        const float4 x = f4_of(v[it]);
        op.put4(r, c, x.x * f, x.y * f, x.z * f, x.w * f);
      } else {
        op.put4(r, c, v[it].x * f, v[it].y * f, v[it].z * f, v[it].w * f);
      }
    }
  }
  // plain fp32 LDS tile with row stride ld
  __device__ __forceinline__ void put_lds(float* s, int ld) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (!live(it)) continue;
      const int idx = threadIdx.x + it * NT;
      if constexpr (sizeof(TS) == 2) {
        *reinterpret_cast<float4*>(s + (idx / V) * ld + 4 * (idx % V)) = f4_of(v[it]);
      } else {
        *reinterpret_cast<float4*>(s + (idx / V) * ld + 4 * (idx % V)) = v[it];
      }
    }
  }
};

// z[e] = x[(e + rot) mod E] for a lane-dependent rot (a multiple of 2 below E), by one select
// stage per bit of rot: static register indices only (a dynamic index would put x in scratch).
template <int E>
__device__ __forceinline__ void rotate(const float (&x)[E], int rot, float (&z)[E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) z[e] = x[e];
#pragma unroll
  for (int bit = E / 2; bit >= 2; bit /= 2) {
    float y[E];
#pragma unroll
    for (int e = 0; e < E; ++e) y[e] = (rot & bit) ? z[(e + bit) % E] : z[e];
#pragma unroll
    for (int e = 0; e < E; ++e) z[e] = y[e];
  }
}

// The transposing load: an R x K fp32 tile (R even) staged as op(c, r) = g[r][c] * ks[r] * cst.
// Slot mapping: G consecutive lanes read 4 consecutive columns each of one source row pair
// (a 128-byte row segment per 8 lanes: coalesced), then the next row pair. Each lane holds rows
// 2j and 2j+1 and writes them as 32-bit pairs of the transposed tile; lane groups q >= 4 write
// their 4 columns in a rotated order so that the 8 groups of one write instruction fall in
// distinct LDS banks (bf16 operand rows of (R + 8)/2 words); without ROT (fewer registers)
// two groups share the banks of each write.
template <int R, int K, int NT, bool ROT = true, class TS = float>
struct RegsT {
  static constexpr int RP = R / 2;
  static constexpr int V = K / 4;
  static constexpr int G = V < 8 ? V : 8;
  static constexpr int IT = (RP * V + NT - 1) / NT;
  Packed4<TS> a[IT], b[IT];  // as stored (fp32, or bf16 expanded when put)
  __device__ __forceinline__ static bool live(int it) {
    return (RP * V) % NT == 0 || (int)threadIdx.x + it * NT < RP * V;
  }
  __device__ __forceinline__ static void slot(int it, int& q, int& j, int& c) {
    const int idx = ((int)threadIdx.x + it * NT) % (RP * V), rest = idx / G;
    q = idx % G;
    j = rest % RP;
    c = 4 * (q + G * (rest / RP));
  }
  // every thread loads (slots past the tile repeat one inside it): no branch around the loads
  __device__ __forceinline__ void fetch(const TS* g, int ldg) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      int q, j, c;
      slot(it, q, j, c);
      a[it] = *reinterpret_cast<const Packed4<TS>*>(lane_ptr(g, 2 * j, ldg, c));
      b[it] = *reinterpret_cast<const Packed4<TS>*>(lane_ptr(g, 2 * j + 1, ldg, c));
    }
  }
  template <int P>
  __device__ __forceinline__ void put(const Op<P>& op, int it, float fa, float fb) const {
    int q, j, c;
    slot(it, q, j, c);
    float xa[4], xb[4];
    if constexpr (sizeof(TS) == 2) {
      const float4 av = f4_of(a[it]), bv = f4_of(b[it]);
      xa[0] = av.x, xa[1] = av.y, xa[2] = av.z, xa[3] = av.w;
      xb[0] = bv.x, xb[1] = bv.y, xb[2] = bv.z, xb[3] = bv.w;
    } else {
      xa[0] = a[it].x, xa[1] = a[it].y, xa[2] = a[it].z, xa[3] = a[it].w;
      xb[0] = b[it].x, xb[1] = b[it].y, xb[2] = b[it].z, xb[3] = b[it].w;
    }
    const int rot = ROT && G == 8 ? 2 * (q / 4) : 0;
    float za[4], zb[4];
    rotate(xa, rot, za);
    rotate(xb, rot, zb);
#pragma unroll
    for (int e = 0; e < 4; ++e) op.put2(c + ((e + rot) & 3), 2 * j, za[e] * fa, zb[e] * fb);
  }
  template <int P>
  __device__ __forceinline__ void put_cols(const Op<P>& op, const float* ks = nullptr, float cst = 1.f) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (!live(it)) continue;
      int q, j, c;
      slot(it, q, j, c);
      put(op, it, (ks ? ks[2 * j] : 1.f) * cst, (ks ? ks[2 * j + 1] : 1.f) * cst);
    }
  }
  // the same with the thread's row pair scaled by (fa, fb): a thread's j is the same in every
  // slot when NT is a multiple of G * R/2
  template <int P>
  __device__ __forceinline__ void put_cols2(const Op<P>& op, float fa, float fb) const {
    static_assert(NT % (G * RP) == 0, "one row pair per thread");
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (live(it)) put(op, it, fa, fb);
    }
  }
  // op(r, c) = g[r][c]: the tile as stored (row layout)
  template <int P>
  __device__ __forceinline__ void put_rows(const Op<P>& op) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (!live(it)) continue;
      int q, j, c;
      slot(it, q, j, c);
      if constexpr (sizeof(TS) == 2) {
        const float4 av = f4_of(a[it]), bv = f4_of(b[it]);
        op.put4(2 * j, c, av.x, av.y, av.z, av.w);
        op.put4(2 * j + 1, c, bv.x, bv.y, bv.z, bv.w);
      } else {
        op.put4(2 * j, c, a[it].x, a[it].y, a[it].z, a[it].w);
        op.put4(2 * j + 1, c, b[it].x, b[it].y, b[it].z, b[it].w);
      }
    }
  }
  // the row pair (2j, 2j+1) this thread holds (put_cols2's rows)
  __device__ __forceinline__ static int pair() { return ((int)threadIdx.x / G) % RP; }
};

template <int R, int K, int NT, int P, class TS>
__device__ __forceinline__ void stage_rows(const Op<P>& op, const TS* g, int ldg, const float* rs = nullptr) {
  Regs<R, K, NT, TS> t;
  t.fetch(g, ldg);
  t.put_rows(op, rs);
}
template <int R, int K, int NT, int P>
__device__ __forceinline__ void stage_cols(const Op<P>& op, const float* g, int ldg, const float* ks = nullptr,
                                           float cst = 1.f) {
  RegsT<R, K, NT> t;
  t.fetch(g, ldg);
  t.put_cols(op, ks, cst);
}

// An R x K tile of a token-major activation (fp32 or bf16, rows past `rows` read as 0), 8
// consecutive values per slot and two consecutive rows per slot, fetched at once and written
// transposed as 32-bit row pairs: op(c, r) = g[r][c].
// An R x K tile of a token-major activation (fp32 or bf16, rows past `rows` read as 0) staged
// transposed: op(c, r) = g[r][c]. As RegsT with 8 consecutive values per lane (16 bytes of
// bf16): G consecutive lanes read one row segment, lane groups rotate their write order so
// the groups of one LDS write instruction fall in distinct banks.
template <int R, int K, int NT, class T>
struct RegsIO {
  static constexpr int RP = R / 2;
  static constexpr int V = K / 8;
  static constexpr int G = V < 8 ? V : 8;
  static constexpr int IT = (RP * V + NT - 1) / NT;
  Raw8<T> x[IT][2];
  int rows;
  __device__ __forceinline__ static bool live(int it) {
    return (RP * V) % NT == 0 || (int)threadIdx.x + it * NT < RP * V;
  }
  __device__ __forceinline__ static void slot(int it, int& q, int& j, int& c) {
    const int idx = ((int)threadIdx.x + it * NT) % (RP * V), rest = idx / G;
    q = idx % G;
    j = rest % RP;
    c = 8 * (q + G * (rest / RP));
  }
  // Every thread loads (slots past the tile repeat one inside it, rows past `rows` >= 1 repeat
  // the last valid row): no branch around the loads and no use of them until put_cols.
  __device__ __forceinline__ void fetch(const T* g, int ldg, int rows_) {
    rows = rows_;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      int q, j, c;
      slot(it, q, j, c);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = 2 * j + h;
        x[it][h].load(lane_ptr(g, r < rows ? r : rows - 1, ldg, c));
      }
    }
  }
  // HI_ONLY (bf16 values into a bf16x3 tile): the high plane only, for P_X3_BEXACT products
  template <int P, bool HI_ONLY = false>
  __device__ __forceinline__ void put_cols(const Op<P>& op) const {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      if (!live(it)) continue;
      int q, j, c;
      slot(it, q, j, c);
      const bool v0 = 2 * j < rows, v1 = 2 * j + 1 < rows;
      const int rot = G == 8 ? 2 * (q / 2) : G == 4 ? 4 * (q / 2) : 0;
      float x0[8], x1[8], z0[8], z1[8];
      x[it][0].get(x0);
      x[it][1].get(x1);
      rotate(x0, rot, z0);
      rotate(x1, rot, z1);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (HI_ONLY) {
          op.put2_hi(c + ((e + rot) & 7), 2 * j, v0 ? z0[e] : 0.f, v1 ? z1[e] : 0.f);
        } else {
          op.put2(c + ((e + rot) & 7), 2 * j, v0 ? z0[e] : 0.f, v1 ? z1[e] : 0.f);
        }
      }
    }
  }
};

// The gates of one thread's row pair (2j, 2j+1) of a chunk -- the rows the thread stages in
// RegsT (RegsT::pair()) -- and of the chunk's last token,
// held in registers: fetch() only issues loads, the accessors derive (no LDS context, no
// barrier). cont: same segment as the token before the chunk (-2 before chunk 0); in_last:
// same segment as the chunk's last token (pallas_tpu_v2.py:226-241).
template <int C>
struct PairGates {
  int s[2], sc, prev;
  float g[2], l[2], bt[2], gc, lc;
  bool first;
  // j: the row pair the thread stages (RegsT::pair())
  __device__ __forceinline__ void fetch(const GdnArgs& A, int b, int h, int n, int j) {
    const size_t tb = (size_t)b * A.Tp + (size_t)n * C;
    const size_t th = (size_t)(b * A.H + h) * A.Tp + (size_t)n * C;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      s[r] = A.segp[tb + 2 * j + r];
      g[r] = A.gam[th + 2 * j + r];
      l[r] = A.gaml[th + 2 * j + r];
      bt[r] = A.bet[th + 2 * j + r];
    }
    sc = A.segp[tb + C - 1];
    gc = A.gam[th + C - 1];
    lc = A.gaml[th + C - 1];
    prev = A.segp[n > 0 ? tb - 1 : tb];
    first = n == 0 && !A.init_state;
  }
  __device__ __forceinline__ int before() const { return first ? -2 : prev; }
  // e^gamma . cont
  __device__ __forceinline__ float grow(int r) const { return s[r] == before() ? expf(g[r] + l[r]) : 0.f; }
  // e^(gamma_C - gamma) . in_last
  __device__ __forceinline__ float kws(int r) const {
    return s[r] == sc ? expf((gc - g[r]) + (lc - l[r])) : 0.f;
  }
  __device__ __forceinline__ float bg(int r) const { return bt[r] * grow(r); }
  __device__ __forceinline__ float carry() const { return sc == before() ? expf(gc + lc) : 0.f; }
};

// The A operand of one wave's 16-row strip over K, fp32 rows of a global tile held raw in
// registers (rows i0 + lane%16, columns 32s + 8 (lane/16) .. +8): fetch() issues the loads,
// product() converts and multiplies (as strip_mma does from memory, with every A fragment
// already in registers).
template <int K>
struct StripA {
  static constexpr int KS = (K + 31) / 32;
  float x[KS][8];
  __device__ __forceinline__ void fetch(const float* g, int ld, int i0) {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      if ((K % 32 == 0) || (32 * s + kg < K)) {
        ld8(lane_ptr(g, i0 + r, ld, 32 * s + kg), x[s]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[s][e] = 0.f;
      }
    }
  }
  // acc[t] += (rs * A)(strip) B(., j0 + 16t ..) for the tiles t < tn; rs scales this lane's
  // A row (i0 + lane%16)
  template <int P, int TN, class BV>
  __device__ __forceinline__ void product(f32x4 (&acc)[TN], const BV& B, int j0, int tn = TN,
                                         float rs = 1.f) const {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bool ok = (K % 32 == 0) || (32 * s + kg < K);
      float xs[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[e] = x[s][e] * rs;
      const Frag<a_prec<P>()> fa = make_frag<a_prec<P>()>(xs);
      tile_row<P, TN>(acc, fa, B, j0, 32 * s + kg, ok, tn);
    }
  }
  // the transposed product: acc[t] += B(i0 + 16t .., .) (strip)^T for the tiles t < TM, B a view
  // or operand tile whose rows are the M index (the strip is the B operand, its rows the N index)
  template <int P, int TM, class AV>
  __device__ __forceinline__ void product_t(f32x4 (&acc)[TM], const AV& B, int i0) const {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bool ok = (K % 32 == 0) || (32 * s + kg < K);
      const Frag<b_prec<P>()> fb = make_frag<b_prec<P>()>(x[s]);
      Frag<a_prec<P>()> fa[TM];
#pragma unroll
      for (int t = 0; t < TM; ++t) fa[t] = ok ? B.template frag<a_prec<P>()>(i0 + 16 * t + r, 32 * s + kg) : zero_frag<a_prec<P>()>();
#pragma unroll
      for (int t = 0; t < TM; ++t) mma<P>(acc[t], fa[t], fb);
    }
  }
  // the strip as stored into an operand tile: op(i0 + r, k) = A(i0 + r, k)
  template <int P>
  __device__ __forceinline__ void put_rows(const Op<P>& op, int i0) const {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      if ((K % 32 == 0) || (32 * s + kg < K)) op.put8(i0 + r, 32 * s + kg, x[s]);
  }
};

// StripA over a token-major activation (fp32 or bf16) held as loaded: rows at or past `rows`
// (>= 1) load the last valid row and read as 0.
template <int K, class T>
struct StripIO {
  static constexpr int KS = (K + 31) / 32;
  Raw8<T> x[KS];
  bool valid;
  __device__ __forceinline__ void fetch(const T* g, int ld, int i0, int rows) {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
    const int rr = i0 + r < rows ? i0 + r : rows - 1;
    valid = i0 + r < rows;
#pragma unroll
    for (int s = 0; s < KS; ++s) x[s].load(lane_ptr(g, rr, ld, (32 * s + kg) % K));
  }
  template <int P, int TN, class BV>
  __device__ __forceinline__ void product(f32x4 (&acc)[TN], const BV& B, int j0, int tn = TN,
                                         float rs = 1.f) const {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
    const float f = valid ? rs : 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const bool ok = (K % 32 == 0) || (32 * s + kg < K);
      float xs[8];
      x[s].get(xs);
#pragma unroll
      for (int e = 0; e < 8; ++e) xs[e] = ok ? xs[e] * f : 0.f;
      const Frag<a_prec<P>()> fa = make_frag<a_prec<P>()>(xs);
      tile_row<P, TN>(acc, fa, B, j0, 32 * s + kg, ok, tn);
    }
  }
};

// One wave's 16 columns [c0, c0 + 16) of a C x D fp32 row tile, staged transposed into the
// wave's own rows c0 .. c0 + 15 of an A(i = column, k = row) operand: lane l holds the row
// pairs (2j, 2j + 1), j = l/4 + 16 it, at columns c0 + 4 (l % 4) .. + 3 (a load covers 16 rows
// of 64 bytes; a write's 64 lanes fall in distinct banks of the bf16 planes). No other wave
// reads those operand rows, so staging and use need no workgroup barrier.
template <int C>
struct StripT {
  static constexpr int RP = C / 2;
  static constexpr int U = (RP * 4 + 63) / 64;
  float4 a[U], b[U];
  __device__ __forceinline__ static int pair(int it) { return ((lane() >> 2) + 16 * it) % RP; }
  __device__ __forceinline__ static bool live(int it) { return RP * 4 >= 64 * (it + 1) || (lane() >> 2) + 16 * it < RP; }
  // every lane loads (lanes past the tile repeat a pair inside it): no branch around the loads
  __device__ __forceinline__ void fetch(const float* g, int ld, int c0) {
    const int col = c0 + 4 * (lane() & 3);
#pragma unroll
    for (int it = 0; it < U; ++it) {
      const int j = pair(it);
      a[it] = *reinterpret_cast<const float4*>(lane_ptr(g, 2 * j, ld, col));
      b[it] = *reinterpret_cast<const float4*>(lane_ptr(g, 2 * j + 1, ld, col));
    }
  }
  // op(c0 + e, r) = g[r][c0 + e] * sc[r] for the held rows r
  template <int P>
  __device__ __forceinline__ void put(const Op<P>& op, int c0, const float* sc) const {
    const int col = c0 + 4 * (lane() & 3);
#pragma unroll
    for (int it = 0; it < U; ++it) {
      if (!live(it)) continue;
      const int j = pair(it);
      const float fa = sc[2 * j], fb = sc[2 * j + 1];
      const float xa[4] = {a[it].x, a[it].y, a[it].z, a[it].w};
      const float xb[4] = {b[it].x, b[it].y, b[it].z, b[it].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) op.put2(col + e, 2 * j, xa[e] * fa, xb[e] * fb);
    }
  }
};

// The fp32 values of a 16-row strip at the accumulator layout of TN 16-column tiles:
// v[t][rr] = g[(i0 + acc_row(rr)) * ld + 16t + acc_col()].
template <int TN>
struct AccVals {
  float v[TN][4];
  __device__ __forceinline__ void fetch(const float* g, int ld, int i0) {
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) v[t][rr] = *lane_ptr(g, i0 + acc_row(rr), ld, 16 * t + acc_col());
  }
  __device__ __forceinline__ void fetch(const uint16_t* g, int ld, int i0) {  // bf16, expanded
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) v[t][rr] = bf2f(*lane_ptr(g, i0 + acc_row(rr), ld, 16 * t + acc_col()));
  }
  __device__ __forceinline__ void clear() {
#pragma unroll
    for (int t = 0; t < TN; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) v[t][rr] = 0.f;
  }
};

template <int R, int D, int NT, class TS>
__device__ __forceinline__ void load_tile(float* s, int LD, const TS* g) {
  Regs<R, D, NT, TS> t;
  t.fetch(g, D);
  t.put_lds(s, LD);
}

// The forward's (v beta)^T operand built from the raw qkv rows of a bf16 I/O conv of 1 to 4 taps
// at C = D = 128 (fuse_v: k_prep skips the v rows). Each thread owns tokens 8 jb .. 8 jb + 7 at
// channels 4m .. 4m + 3, whose conv reads raw rows 8 jb - 3 .. 8 jb + 7: they land during the
// inverse, and the conv and SiLU run as the operand is put, in k_prep's fp32 arithmetic (the same
// values k_prep would store), one 16-byte write per channel and plane. Lane l of wave w:
// m = 16 (w % 2) + 2 (l / 8) + l % 2, jb = 4 (w / 2) + (l / 2) % 4, so that any 16 consecutive
// lanes write 16 distinct 16-byte bank groups (row stride 272 bytes) and 16 lanes read 128
// contiguous bytes of a row. The unit's conv weights go through LDS (lag threadIdx.x / D).
template <int C, int D, int NT>
struct RawV {
  static_assert(C == 128 && D == 128 && NT == 512, "the lane map of C = D = 128");
  Raw4<uint16_t> raw[11];
  float wt;
  __device__ __forceinline__ static int chan4() {
    return 4 * (16 * (wave() & 1) + 2 * (lane() >> 3) + (lane() & 1));
  }
  __device__ __forceinline__ static int row0() { return 8 * (4 * (wave() >> 1) + ((lane() >> 1) & 3)); }
  __device__ __forceinline__ void fetch(const GdnArgs& A, int b, int h, int n) {
    const uint16_t* x = reinterpret_cast<const uint16_t*>(A.qkv);
    const int c0 = (2 * A.Hk + h) * D, c = chan4(), r0 = row0();
#pragma unroll
    for (int i = 0; i < 11; ++i) raw[i].load(halo_row<uint16_t>(A, x, b, n * C + r0 - 3 + i, c0 + c));
    const int lag = threadIdx.x / D;  // lags past the taps read lag 0's (a weight of zero when put)
    wt = A.conv_w[(size_t)(lag < A.taps ? A.taps - 1 - lag : A.taps - 1) * A.W + c0 + threadIdx.x % D];
  }
  __device__ __forceinline__ void put_weights(float* sw, const GdnArgs& A) const {
    sw[threadIdx.x] = (int)threadIdx.x / D < A.taps ? wt : 0.f;
  }
  // after put_weights and a barrier
  template <int P>
  __device__ __forceinline__ void put_cols(const Op<P>& op, const Ctx<C>& cx, const float* sw, const GdnArgs& A,
                                           int n) const {
    const int c = chan4(), r0 = row0();
    int sr[11];  // ids of rows r0 - 3 .. r0 + 7 (rows before the chunk: the context's halo ids)
#pragma unroll
    for (int i = 0; i < 11; ++i) {
      const int r = r0 - 3 + i;
      sr[i] = i >= 3 ? cx.seg[r] : *(r >= 0 ? &cx.seg[r] : &cx.hseg[-1 - r]);
    }
    bool keep[8][4];  // keep[i][L]: token r0 + i reads row r0 + i - L
    bool live[8];     // token r0 + i is not padding
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int t = n * C + r0 + i;
      const int st = t < A.T ? sr[3 + i] : 0;
      live[i] = st > 0;
#pragma unroll
      for (int L = 1; L <= 3; ++L) keep[i][L] = L < A.taps && (t - L >= 0 || A.init_conv) && sr[3 + i - L] == st;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // channel c + e, as k_prep: z = sum over lags of keep * x[t-L] * w[K-1-L]
      float wl[4], x[11], v[8];
#pragma unroll
      for (int L = 0; L < 4; ++L) wl[L] = sw[L * D + c + e];
#pragma unroll
      for (int i = 0; i < 11; ++i) x[i] = raw[i].elem(e);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float z = x[3 + i] * wl[0];
#pragma unroll
        for (int L = 1; L <= 3; ++L) z = keep[i][L] ? z + x[3 + i - L] * wl[L] : z;
        v[i] = (live[i] ? z * sigmoid_io<uint16_t>(z) : 0.f) * cx.beta[r0 + i];
      }
      op.put8(c + e, r0, v);
    }
  }
};

// ---------------------------------------------------------------- k_chunk
// Persistent over the (row, head, chunk) units as k_out; C/16 waves (one 16-row strip each).
// MODE 0 (forward): writes w and u; MODE 2: also T (kept as a residual). MODE 1 (backward
// recompute): writes T and v_new = u - w S_before, computed as T (v beta - kbe S_before) (one
// state-path product and one with T instead of w, u and w S); MODE 3: v_new from the saved T
// (no L, no inverse). LDS: T in fp32 (the inverse runs in place), one operand region reused
// for k, kbe^T, (v beta)^T, S^T and Y^T (and T^T during the inverse). The next unit's context
// and k rows are loaded at this unit's start and end; the forward's k (again) and v, and the
// backward's S and k strip, during the inverse; the backward's v after it (held across the
// inverse, it would spill). DBL: the inverse's diagonal blocks by doubling (else by substitution;
// a template argument: both forms in one kernel take 17 more VGPRs and spill in MODE 1). FV: the
// forward's v built from the raw rows (RawV) instead of read from k_prep's rows.
template <int C, int D, int PI, int PS, int MODE, bool DBL, bool FV = false>
__global__ __launch_bounds__(C * 4) void k_chunk(GdnArgs A) {
  constexpr bool FWD = MODE == 0 || MODE == 2;  // writes w and u (else v_new)
  constexpr bool LOAD_T = MODE == 3;            // T from the residuals
  constexpr bool STORE_T = MODE == 1 || MODE == 2;
  constexpr int NT = C * 4;
  constexpr int M = C > D ? C : D;
  constexpr int LT = M + 4;
  using TB = OpTile<PI, M, M>;
  constexpr int RB = TB::BYTES > C * LT * 4 ? TB::BYTES : C * LT * 4;  // also T^T during the inverse
  __shared__ __align__(16) float sT[C * LT];
  __shared__ __align__(16) char sB[RB];
  __shared__ Ctx<C> cx;
  __shared__ __align__(16) float sW[FV ? 4 * D : 4];  // FV: the unit's conv weights
  static_assert(!FV || FWD, "FV: the forward modes");
  GDN_POISON_LDS(sT, sB, cx, sW);
  const int w = wave(), i0 = 16 * w;
  const Op<PI> ob = TB::at(sB);
  const int total = A.B * A.H * A.N;
  CtxRaw<C, FV> rc;
  RegsT<C, D, NT> kk;  // k: staged as rows (A and B of k k^T), then as kbe^T
  {
    const UnitIx<CHUNKS_DOWN> x(A, blockIdx.x);
    rc.fetch(A, x.b, x.h, x.n);
    kk.fetch(A.kn + hoff(A, x.b, x.hk, A.Hk, x.n, C, D), D);
  }
  for (int u = blockIdx.x; u < total; u += gridDim.x) {
    const UnitIx<CHUNKS_DOWN> x(A, u);
    const UnitIx<CHUNKS_DOWN> y(A, u + gridDim.x < total ? u + gridDim.x : u);  // the next unit (or this one again)
    const size_t off = hoff(A, x.b, x.h, A.H, x.n, C, D);
    TinvT<PI>* tg = tinv_ptr<PI>(A) + ((size_t)(x.b * A.H + x.h) * A.N + x.n) * C * C;
    rc.commit(cx);
    if constexpr (!LOAD_T) kk.put_rows(ob);
    rc.fetch(A, y.b, y.h, y.n);
    std::conditional_t<FV, RawV<C, D, NT>, RegsT<C, D, NT>> vc;  // this unit's (v beta)^T source (forward)
    RegsT<D, D, NT, true, StateT<PS>> sc;  // S_before, its strip of k and its v at the accumulator layout (backward)
    StripA<D> ks;
    AccVals<D / 16> va;
    if constexpr (LOAD_T) {
      load_tile<C, C, NT>(sT, LT, tg);
      sc.fetch(states_ptr<PS>(A) + ((size_t)(x.b * A.H + x.h) * A.N + x.n) * D * D, D);
      ks.fetch(A.kn + hoff(A, x.b, x.hk, A.Hk, x.n, C, D), D, i0);
      va.fetch(A.vv + off, D, i0);
    }
    __syncthreads();
    derive_ctx<C, NT>(cx);
    __syncthreads();
    if constexpr (!LOAD_T) {
      {  // L = strict(beta_i (k k^T)_ij D_ij): tiles on and below the diagonal only
        f32x4 acc[C / 16];
        zero(acc);
        strip_mma<PI, D, C / 16>(acc, ob, i0, ob, 0, 0, D, w + 1);
        // every tile's values first, then the stores: the single stores' memory clobber would
        // otherwise keep the next tile's context reads (LDS) behind them
        const StripDecay<C> sd(cx, i0);
        float bt[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) bt[rr] = cx.beta[i0 + acc_row(rr)];
#pragma unroll
        for (int t = 0; t < C / 16; ++t) {
          float d[4];
          sd.tile(cx, i0, t, w, d);
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            acc[t][rr] = i0 + acc_row(rr) > 16 * t + acc_col() ? bt[rr] * acc[t][rr] * d[rr] : 0.f;
        }
#pragma unroll
        for (int t = 0; t < C / 16; ++t)
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) lds_st(sT + (i0 + acc_row(rr)) * LT + 16 * t + acc_col(), acc[t][rr]);
      }
      if constexpr (!FWD) {  // in flight during the inverse
        sc.fetch(states_ptr<PS>(A) + ((size_t)(x.b * A.H + x.h) * A.N + x.n) * D * D, D);
        ks.fetch(A.kn + hoff(A, x.b, x.hk, A.Hk, x.n, C, D), D, i0);
      }
      if constexpr (FWD) {  // k again and v, in flight during the inverse
        kk.fetch(A.kn + hoff(A, x.b, x.hk, A.Hk, x.n, C, D), D);
        if constexpr (FV) vc.fetch(A, x.b, x.h, x.n);
        else vc.fetch(A.vv + off, D);
      }
      __syncthreads();
      invert_unit_lower<C, PI>(sT, LT, reinterpret_cast<float*>(sB), DBL);
      if constexpr (!FWD) {
        va.fetch(A.vv + off, D, i0);
      }
    }
    if constexpr (!FWD) {  // v_new = T (v beta - kbe S_before): one state-path product, one with T
      f32x4 yv[D / 16];
      zero(yv);
      sc.put_cols(ob);  // S^T
      __syncthreads();
      ks.template product<PS>(yv, ob, 0, D / 16, -cx.bg[i0 + (lane() & 15)]);  // - kbe S
#pragma unroll
      for (int t = 0; t < D / 16; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) yv[t][rr] += va.v[t][rr] * cx.beta[i0 + acc_row(rr)];
      __syncthreads();
#pragma unroll
      for (int t = 0; t < D / 16; ++t)  // Y^T: B(c, j) = Y[c][j]
        ob.put4(16 * t + acc_col(), i0 + acc_row(0), yv[t][0], yv[t][1], yv[t][2], yv[t][3]);
      kk.fetch(A.kn + hoff(A, y.b, y.hk, A.Hk, y.n, C, D), D);  // the next unit's k
      __syncthreads();
      f32x4 vn[D / 16];
      zero(vn);
      strip_mma<PI, C, D / 16>(vn, krow(sT, LT), i0, ob, 0, 0, tri_end<C>(i0));
      if constexpr (STORE_T) {  // for k_bwd_local (fetch_lower): the tiles on and below the diagonal
#pragma unroll 2
        for (int idx = threadIdx.x; idx < C * C / 4; idx += NT) {
          const int r = idx / (C / 4), c = 4 * (idx % (C / 4));
          if ((c >> 4) <= (r >> 4)) {  // the lower triangle (the rest of sT is scratch)
            const float4 t = *reinterpret_cast<const float4*>(sT + r * LT + c);
            if constexpr (sizeof(TinvT<PI>) == 2) {
              const float v[4] = {c <= r ? t.x : 0.f, c + 1 <= r ? t.y : 0.f, c + 2 <= r ? t.z : 0.f, c + 3 <= r ? t.w : 0.f};
              st4_io(tg + r * C + c, v);
            } else {
              *reinterpret_cast<float4*>(tg + r * C + c) =
                  make_float4(c <= r ? t.x : 0.f, c + 1 <= r ? t.y : 0.f, c + 2 <= r ? t.z : 0.f, c + 3 <= r ? t.w : 0.f);
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < D / 16; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) A.vnew[off + (i0 + acc_row(rr)) * D + 16 * t + acc_col()] = vn[t][rr];
      __syncthreads();  // cx, sT and the operand region are rewritten by the next unit
      continue;
    }
    f32x4 aw[D / 16], au[D / 16];
    zero(aw);
    zero(au);
    kk.put_cols(ob, cx.bg);  // kbe^T
    if constexpr (FV) vc.put_weights(sW, A);
    __syncthreads();
    strip_mma<PI, C, D / 16>(aw, krow(sT, LT), i0, ob, 0, 0, tri_end<C>(i0));
#pragma unroll
    for (int t = 0; t < D / 16; ++t)  // w now: its stores drain during the u product
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) A.ww[off + (size_t)(i0 + acc_row(rr)) * D + 16 * t + acc_col()] = aw[t][rr];
    __syncthreads();
    if constexpr (FV) vc.put_cols(ob, cx, sW, A, x.n);  // (v beta)^T
    else vc.put_cols(ob, cx.beta);
    __syncthreads();
    strip_mma<PI, C, D / 16>(au, krow(sT, LT), i0, ob, 0, 0, tri_end<C>(i0));
    // the next unit's k before this unit's stores: waiting for it later (vmcnt counts in issue
    // order, stores included) then does not wait for the stores
    kk.fetch(A.kn + hoff(A, y.b, y.hk, A.Hk, y.n, C, D), D);
    if constexpr (STORE_T) {
      for (int idx = threadIdx.x; idx < C * C; idx += NT)  // lower triangle (the rest is scratch)
        stf(tg + idx, idx % C <= idx / C ? sT[(idx / C) * LT + idx % C] : 0.f);
    }
#pragma unroll
    for (int t = 0; t < D / 16; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) A.uu[off + (size_t)(i0 + acc_row(rr)) * D + 16 * t + acc_col()] = au[t][rr];
    __syncthreads();  // cx, sT and the operand region are rewritten by the next unit
  }
}

// ---------------------------------------------------------------- scan partition
// carry of chunk c: its last token continues the segment of the token before the chunk (-2
// before chunk 0, or token 0's id with an initial state). Where a chunk does not carry, the state after it does not depend on the state
// before it (its last segment starts inside it and reads no earlier state), and the state
// gradient entering it does not depend on the one after it (the rows that read the earlier
// state, and so feed that gradient, are in another segment than the rows that write the later
// state: their coupling terms are exact zeros). The scans split each chain there into
// independent chunk ranges (bitwise equal to the unsplit chain).
template <int C>
__device__ __forceinline__ bool chunk_carries(const GdnArgs& A, int b, int c) {
  const int32_t* sp = A.segp + (size_t)b * A.Tp;
  const int before = c == 0 ? (A.init_state ? sp[0] : -2) : sp[(size_t)c * C - 1];
  return sp[(size_t)c * C + C - 1] == before;
}
// The first chunk s in [q, N) where a range starts, or N; forward ranges start at chunk 0 and
// after chunks that do not carry, backward ranges at chunk 0 and at chunks that do not carry. One candidate per thread, then the workgroup minimum (red: NT/64 ints of LDS).
// Called by every thread of the workgroup.
template <int C, int NT, bool FWD>
__device__ __forceinline__ int part_start(const GdnArgs& A, int b, int q, int* red) {
  for (int base = q; base < A.N; base += NT) {
    const int s = base + (int)threadIdx.x;
    bool hit = false;
    if (s < A.N) hit = s == 0 || (FWD ? !chunk_carries<C>(A, b, s - 1) : !chunk_carries<C>(A, b, s));
    int m = hit ? s : A.N;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = min(m, __shfl_xor(m, off));
    if (lane() == 0) red[wave()] = m;
    __syncthreads();
    int best = A.N;
    for (int i = 0; i < NT / 64; ++i) best = min(best, red[i]);
    __syncthreads();
    if (best < A.N) return best;
  }
  return A.N;
}

// scan workgroup id -> (part, row * heads + head, Dv tile): part-major in dispatch order (the
// first ranges, never empty, start first), then XCD-remapped so a head's tiles share an L2
struct ScanIx {
  int part, bh, tile;
  __device__ __forceinline__ ScanIx(const GdnArgs& A) {
    const int chains = A.B * A.H * A.ntiles;
    part = blockIdx.x / chains;
    const int id = xcd_remap(blockIdx.x % chains, chains);
    tile = id % A.ntiles;
    bh = id / A.ntiles;
  }
};

// ---------------------------------------------------------------- k_scan_fwd
// grid B*H*(D/DVT) (XCD-remapped), max(C,D)/16 waves; chunks in order (pallas_tpu_v2.py:254-269).
// The products run transposed, v_new^T = u^T - S^T w^T and S^T = carry S^T + v_new^T (k kws),
// so that an accumulator lane holds 4 consecutive value columns of one token (one dk row of
// S): u is loaded and v_new and the states are stored as 16-byte vectors. S^T lives in the
// accumulators of waves < D/16 (wave w: dk columns 16w .. 16w + 15, all DVT value rows). None
// of a chunk step's global inputs depends on S, so each is held in registers and refilled
// with the next chunk's values as soon as it has been used: those loads run during the rest of
// the step (its products and barriers) instead of stalling the next one. Two barriers per step.
template <int C, int D, int DVT, int NT>
struct ScanFwdIn {
  PairGates<C> gt;     // kws of the thread's k rows, and the carry
  RegsT<C, D, NT> k;   // k rows, staged as (k kws)^T
  StripA<D> wa;        // w rows of this wave's 16 tokens (the B operand of S^T w^T)
  float4 u[DVT / 16];  // u[token][j0 + 16t + 4 (lane/16) ..] of the lane's token
  __device__ __forceinline__ void fetch_k(const GdnArgs& A, int b, int hk, int n) {
    k.fetch(A.kn + hoff(A, b, hk, A.Hk, n, C, D), D);
  }
  // waves past the C/16 strips load a strip they do not use: no branch around the loads
  __device__ __forceinline__ void fetch_w(const GdnArgs& A, int b, int h, int n) {
    wa.fetch(A.ww + hoff(A, b, h, A.H, n, C, D), D, 16 * (wave() % (C / 16)));
  }
  __device__ __forceinline__ void fetch_u(const GdnArgs& A, int b, int h, int n, int j0) {
    const float* g = A.uu + hoff(A, b, h, A.H, n, C, D) + (size_t)(16 * (wave() % (C / 16)) + acc_col()) * D + j0 +
                     4 * (lane() >> 4);
#pragma unroll
    for (int t = 0; t < DVT / 16; ++t) u[t] = *reinterpret_cast<const float4*>(g + 16 * t);
  }
};

template <int C, int D, int DVT, int PI, int PS>
__global__ __launch_bounds__((C > D ? C : D) * 4) void k_scan_fwd(GdnArgs A) {
  constexpr int NT = (C > D ? C : D) * 4;
  constexpr int NW = NT / 64;  // wave conditions below are compile-time when every wave takes part
  constexpr int TJ = DVT / 16;
  using TS = OpTile<PI, DVT, D>;   // S^T: A(i = j, k = dk)
  using TK = OpTile<PI, D, C>;     // (k kws): B(k = c, j = dk), stored as (k kws)^T
  using TV = OpTile<PI, DVT, C>;   // v_new^T: A(i = j, k = c)
  __shared__ __align__(16) char sS[TS::BYTES];
  __shared__ __align__(16) char sK[TK::BYTES];
  __shared__ __align__(16) char sV[TV::BYTES];
  const Op<PI> os = TS::at(sS), ok = TK::at(sK), ov = TV::at(sV);
  __shared__ int red[NW];
  GDN_POISON_LDS(sS, sK, sV, red);
  const ScanIx ix(A);
  const int tile = ix.tile, bh = ix.bh, part = ix.part;
  const int h = bh % A.H, b = bh / A.H, hk = h / A.ratio;
  const int j0 = tile * DVT;
  const int w = wave();
  const int jl = 4 * (lane() >> 4);  // the lane's first value column within a 16-column tile
  // this workgroup's chunks [n0, n1); from n0 - 1 (not stored) when the range starts after chunk 0
  const int n0 = part_start<C, NT, true>(A, b, (int)((long)part * A.N / A.parts), red);
  const int n1 = part_start<C, NT, true>(A, b, (int)((long)(part + 1) * A.N / A.parts), red);
  if (n0 >= n1) return;
  const int nb = n0 > 0 ? n0 - 1 : 0;
  f32x4 accS[TJ];  // accS[t][rr] = S[16w + acc_col()][j0 + 16t + jl + rr]
  zero(accS);
  if (n0 == 0 && A.init_state && (NW == D / 16 || w < D / 16)) {  // a continued sequence: S before chunk 0
    const float* s0 = A.init_state + (size_t)bh * D * D + (size_t)(16 * w + acc_col()) * D + j0 + jl;
#pragma unroll
    for (int t = 0; t < TJ; ++t) {
      const float4 v = *reinterpret_cast<const float4*>(s0 + 16 * t);
      accS[t] = f32x4{v.x, v.y, v.z, v.w};
    }
  }
  ScanFwdIn<C, D, DVT, NT> in;
  in.gt.fetch(A, b, h, nb, RegsT<C, D, NT>::pair());
  in.fetch_k(A, b, hk, nb);
  in.fetch_w(A, b, h, nb);
  in.fetch_u(A, b, h, nb, j0);
  for (int n = nb; n < n1; ++n) {
    const int nx = n + 1 < n1 ? n + 1 : n;  // the last step refetches its own chunk (unused)
    const bool emit = n >= n0;              // the replayed chunk n0 - 1 only rebuilds the state
    if (NW == D / 16 || w < D / 16) {
      const int dk = 16 * w + acc_col();
      const size_t so = ((size_t)bh * A.N + n) * D * D + (size_t)dk * D + j0 + jl;
      StateT<PS>* sg = states_ptr<PS>(A) + so;
#pragma unroll
      for (int t = 0; t < TJ; ++t) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) os.put(16 * t + jl + rr, dk, accS[t][rr]);
        const float v[4] = {accS[t][0], accS[t][1], accS[t][2], accS[t][3]};
        if (emit) st4_io(sg + 16 * t, v);
        if constexpr (sizeof(StateT<PS>) == 2) {  // the final state's fp32 source
          if (emit && n == A.N - 1 && A.s_last) st4_io(A.s_last + ((size_t)bh * D + dk) * D + j0 + jl + 16 * t, v);
        }
      }
    }
    const float carry = in.gt.carry();
    __syncthreads();
    if (NW == C / 16 || w < C / 16) {  // v_new^T = u^T - S^T w^T for the wave's 16 tokens
      f32x4 acc[TJ];
      zero(acc);
      in.wa.template product_t<PS>(acc, os, 0);
      in.fetch_w(A, b, h, nx);
      const int i = 16 * w + acc_col();
      float* vg = A.vnew + hoff(A, b, h, A.H, n, C, D) + (size_t)i * D + j0 + jl;
#pragma unroll
      for (int t = 0; t < TJ; ++t) {
        const float vn[4] = {in.u[t].x - acc[t][0], in.u[t].y - acc[t][1], in.u[t].z - acc[t][2], in.u[t].w - acc[t][3]};
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) ov.put(16 * t + jl + rr, i, vn[rr]);
        if (emit) *reinterpret_cast<float4*>(vg + 16 * t) = make_float4(vn[0], vn[1], vn[2], vn[3]);
      }
      in.fetch_u(A, b, h, nx, j0);
    }
    // (k kws)^T after the product, so one wave's staging overlaps the other's MFMA work
    in.k.put_cols2(ok, in.gt.kws(0), in.gt.kws(1));
    in.fetch_k(A, b, hk, nx);
    in.gt.fetch(A, b, h, nx, RegsT<C, D, NT>::pair());
    __syncthreads();
    if (NW == D / 16 || w < D / 16) {  // S^T = carry S^T + v_new^T (k kws)
#pragma unroll
      for (int t = 0; t < TJ; ++t) accS[t] *= carry;
      col_mma<PI, C, TJ>(accS, ov, 0, ok, 16 * w);
    }
    // no barrier here: the next step's first writes go to the S tile, which this product
    // does not read, and the k and v_new tiles are rewritten only after its first barrier
  }
}

// ---------------------------------------------------------------- k_scan_fwd_split
// The forward scan at C = D = 128 with its two products chained in registers. Two compute
// waves each own 16 value columns of the 32-column Dv tile: S[:, cols] (Dk x 16, 8 accumulator
// tiles, rows dk) and v_new[:, cols] (C x 16, 8 tiles, rows tokens). Per chunk:
//   P1  v_new = u + (-w) S             A: -w (LDS, rows tokens), B: S from the accumulators
//   P2  S = carry S + k^T (kws v_new)  A: k^T (LDS, rows dk), B: v_new from the accumulators,
//                                      its rows (tokens) scaled by kws
// A product's B operand has the contraction index along the other product's accumulator rows:
// two accumulator tiles (rows 0-15, 16-31) become one 32-deep B fragment by one permlane32 and
// one permlane16 swap per register (lane group kq then holds rows 8kq .. 8kq + 7 of its
// column), so neither result goes through LDS and the products need no barrier between them.
// The other six waves stage the LDS operands a product ahead: k^T of chunk n during P1 of
// chunk n, -w, u^T and the gates of chunk n + 1 during P2 of chunk n, each from registers loaded
// one product earlier. They also store the states: a compute wave leaves S before chunk n in
// its columns of the u^T buffer once it has read u from there, and in P2 each loader thread
// stores the values it then overwrites with the next u^T. Two barriers per chunk. Same chunk
// ranges, replays and outputs as k_scan_fwd.
struct ScanSplitBuf {
  static constexpr int C = 128, D = 128, DVT = 32, LU = C + 4;
};

// B fragment values (rows 8 (lane/16) .. + 7 of the 32-row contraction step, column lane % 16)
// from accumulator tiles t0 (rows 0-15) and t1 (rows 16-31)
__device__ __forceinline__ void acc_pair_to_b(const f32x4& t0, const f32x4& t1, float (&v)[8]) {
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) {
    // (the element values are copied out first: __builtin_bit_cast of a vector element
    // subscript reads element 0 whatever the index, with this compiler)
    const float a = t0[rr], c = t1[rr];
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(c), false, false);
    const unsigned p0 = p[0], p1 = p[1];
    const auto q = __builtin_amdgcn_permlane16_swap(p0, p1, false, false);
    const unsigned q0 = q[0], q1 = q[1];
    v[rr] = __uint_as_float(q0);
    v[4 + rr] = __uint_as_float(q1);
  }
}

// acc[t] += A(16 t + lane % 16, k) B(k, lane % 16) over a 128-deep contraction: A from an LDS
// operand tile (8 row tiles), B from the accumulator tiles bsrc (two per 32-deep step). Each
// step's eight A fragments are read one step ahead, so the LDS latency runs under the previous
// step's MFMAs.
template <int P, class OP>
__device__ __forceinline__ void split_product(f32x4 (&acc)[8], const OP& a, const f32x4 (&bsrc)[8],
                                              const float* bscale = nullptr) {
  const int r = lane() & 15, kg = (lane() >> 4) << 3;
  Frag<a_prec<P>()> fa[2][8];
#pragma unroll
  for (int t = 0; t < 8; ++t) fa[0][t] = a.template frag<a_prec<P>()>(16 * t + r, kg);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    if (s + 1 < 4) {
#pragma unroll
      for (int t = 0; t < 8; ++t) fa[(s + 1) & 1][t] = a.template frag<a_prec<P>()>(16 * t + r, 32 * (s + 1) + kg);
    }
    // the scheduler would otherwise sink these reads next to their MFMAs (register pressure)
    __builtin_amdgcn_sched_barrier(0);
    float bv[8];
    acc_pair_to_b(bsrc[2 * s], bsrc[2 * s + 1], bv);
    if (bscale) {  // B(k, .) scaled by bscale[k]: the lane's 8 contraction rows
      const float4 s0 = *reinterpret_cast<const float4*>(bscale + 32 * s + kg);
      const float4 s1 = *reinterpret_cast<const float4*>(bscale + 32 * s + kg + 4);
      bv[0] *= s0.x; bv[1] *= s0.y; bv[2] *= s0.z; bv[3] *= s0.w;
      bv[4] *= s1.x; bv[5] *= s1.y; bv[6] *= s1.z; bv[7] *= s1.w;
    }
    const Frag<b_prec<P>()> fb = make_frag<b_prec<P>()>(bv);
#pragma unroll
    for (int t = 0; t < 8; ++t) mma<P>(acc[t], fa[s & 1][t], fb);
  }
}

template <int PI, int PS>
__global__ __launch_bounds__(512) void k_scan_fwd_split(GdnArgs A) {
  constexpr int C = 128, D = 128, DVT = 32, NT = 512, LU = C + 4;
  constexpr int NL = NT - 128;      // loader threads (waves 2 .. 7)
  using TW = OpTile<PI, C, D>;      // -w: A(i = token, k = dk)
  using TK = OpTile<PI, D, C>;      // k^T: A(i = dk, k = token)
  __shared__ __align__(16) char sW[TW::BYTES];
  __shared__ __align__(16) char sK[TK::BYTES];
  __shared__ __align__(16) float sU[DVT * LU];  // u^T: [value column][token]
  __shared__ __align__(16) float skws[2][C];    // kws per token, by chunk parity
  __shared__ float scarry[2];
  __shared__ int red[NT / 64];
  GDN_POISON_LDS(sW, sK, sU, skws, scarry, red);
  const Op<PI> ow = TW::at(sW), okt = TK::at(sK);
  const ScanIx ix(A);
  const int tile = ix.tile, bh = ix.bh, part = ix.part;
  const int h = bh % A.H, b = bh / A.H, hk = h / A.ratio;
  const int j0 = tile * DVT;
  const int w = wave(), l = lane();
  const int n0 = part_start<C, NT, true>(A, b, (int)((long)part * A.N / A.parts), red);
  const int n1 = part_start<C, NT, true>(A, b, (int)((long)(part + 1) * A.N / A.parts), red);
  if (n0 >= n1) return;
  const int nb = n0 > 0 ? n0 - 1 : 0;
  const bool compute = w < 2;  // wave-uniform
  const int lt = (int)threadIdx.x - 128;  // loader thread index (>= 0 in waves 2 .. 7)
  // ---- loader state: the next operands in registers
  float4 wr[11];            // -w: 4096 float4 slots over 384 threads
  float4 ka[6], kb[6];      // k rows 2j, 2j+1 at 4 dk columns: 2048 slots
  float4 ur[3];             // u: 1024 float4 slots
  int gs = 0, gsc = 0, gprev = 0;
  float gg = 0.f, gl = 0.f, ggc = 0.f, glc = 0.f;
  auto fetch_w = [&](int n) {
    const float* g = A.ww + hoff(A, b, h, A.H, n, C, D);
#pragma unroll
    for (int it = 0; it < 11; ++it) {
      const int idx = min(lt + it * NL, 4095);
      wr[it] = *reinterpret_cast<const float4*>(lane_ptr(g, idx >> 5, D, 4 * (idx & 31)));
    }
  };
  auto fetch_u = [&](int n) {
    const float* g = A.uu + hoff(A, b, h, A.H, n, C, D) + j0;
#pragma unroll
    for (int it = 0; it < 3; ++it) {
      const int idx = min(lt + it * NL, 1023);
      ur[it] = *reinterpret_cast<const float4*>(lane_ptr(g, idx >> 3, D, 4 * (idx & 7)));
    }
  };
  auto fetch_k = [&](int n) {
    const float* g = A.kn + hoff(A, b, hk, A.Hk, n, C, D);
#pragma unroll
    for (int it = 0; it < 6; ++it) {
      const int idx = min(lt + it * NL, 2047), q = idx & 7, rest = idx >> 3, j = rest & 63;
      const int c = 4 * (q + 8 * (rest >> 6));
      ka[it] = *reinterpret_cast<const float4*>(lane_ptr(g, 2 * j, D, c));
      kb[it] = *reinterpret_cast<const float4*>(lane_ptr(g, 2 * j + 1, D, c));
    }
  };
  // the gates of chunk n: token lt's segment and gamma (lt < C), the chunk's last token and the
  // token before it
  auto fetch_g = [&](int n) {
    const size_t tb = (size_t)b * A.Tp + (size_t)n * C, th = (size_t)(b * A.H + h) * A.Tp + (size_t)n * C;
    const int t = lt < C ? lt : C - 1;
    gs = A.segp[tb + t];
    gg = A.gam[th + t];
    gl = A.gaml[th + t];
    gsc = A.segp[tb + C - 1];
    ggc = A.gam[th + C - 1];
    glc = A.gaml[th + C - 1];
    gprev = A.segp[n > 0 ? tb - 1 : tb];
  };
  auto put_gates = [&](int n) {  // kws and carry of chunk n into the parity buffers
    const int before = (n == 0 && !A.init_state) ? -2 : gprev;
    if (lt < C) skws[n & 1][lt] = gs == gsc ? expf((ggc - gg) + (glc - gl)) : 0.f;
    if (lt == 0) scarry[n & 1] = gsc == before ? expf(ggc + glc) : 0.f;
  };
  auto put_w = [&]() {
#pragma unroll
    for (int it = 0; it < 11; ++it) {
      const int idx = lt + it * NL;
      if (idx < 4096) ow.put4(idx >> 5, 4 * (idx & 31), -wr[it].x, -wr[it].y, -wr[it].z, -wr[it].w);
    }
  };
  auto store_s = [&](int n) {  // S before chunk n, from sU, where put_u writes next
    StateT<PS>* sg = states_ptr<PS>(A) + ((size_t)bh * A.N + n) * D * D + j0;
#pragma unroll
    for (int it = 0; it < 3; ++it) {
      const int idx = lt + it * NL;
      if (idx < 1024) {
        const int dk = idx >> 3, c = 4 * (idx & 7);
        if constexpr (sizeof(StateT<PS>) == 2) {  // and the final state's fp32 source
          const float v[4] = {sU[(c + 0) * LU + dk], sU[(c + 1) * LU + dk], sU[(c + 2) * LU + dk],
                              sU[(c + 3) * LU + dk]};
          st4_io(sg + (unsigned)(dk * D + c), v);
          if (n == A.N - 1 && A.s_last) st4_io(A.s_last + (size_t)bh * D * D + j0 + (unsigned)(dk * D + c), v);
        } else {
          const float4 v = make_float4(sU[(c + 0) * LU + dk], sU[(c + 1) * LU + dk], sU[(c + 2) * LU + dk],
                                       sU[(c + 3) * LU + dk]);
          *reinterpret_cast<float4*>(sg + (unsigned)(dk * D + c)) = v;
        }
      }
    }
  };
  auto put_u = [&]() {
#pragma unroll
    for (int it = 0; it < 3; ++it) {
      const int idx = lt + it * NL;
      if (idx < 1024) {
        const int tk = idx >> 3, c = 4 * (idx & 7);
        sU[(c + 0) * LU + tk] = ur[it].x;
        sU[(c + 1) * LU + tk] = ur[it].y;
        sU[(c + 2) * LU + tk] = ur[it].z;
        sU[(c + 3) * LU + tk] = ur[it].w;
      }
    }
  };
  auto put_k = [&]() {  // k^T: op(dk, token) = k[token][dk] as 32-bit token pairs (kws is applied
                        // to v_new's rows on the compute side)
#pragma unroll
    for (int it = 0; it < 6; ++it) {
      const int idx = lt + it * NL;
      if (idx < 2048) {
        const int q = idx & 7, rest = idx >> 3, j = rest & 63, c = 4 * (q + 8 * (rest >> 6));
        okt.put2(c + 0, 2 * j, ka[it].x, kb[it].x);
        okt.put2(c + 1, 2 * j, ka[it].y, kb[it].y);
        okt.put2(c + 2, 2 * j, ka[it].z, kb[it].z);
        okt.put2(c + 3, 2 * j, ka[it].w, kb[it].w);
      }
    }
  };
  // Each role runs its own loop (their registers are then never live together), with the same
  // barriers: one before the first chunk, two per chunk.
  if (compute) {
    const int jt = w & 1;          // the wave's 16 value columns
    const int col = j0 + 16 * jt;  // first value column of the wave
    f32x4 accS[8];  // S[16 dt + 4 (lane/16) + rr][col + lane % 16]
    f32x4 accV[8];  // v_new[16 rt + 4 (lane/16) + rr][col + lane % 16]
    zero(accS);
    if (n0 == 0 && A.init_state) {
      const float* s0 = A.init_state + (size_t)bh * D * D + col + acc_col();
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) accS[dt][rr] = s0[(size_t)(16 * dt + acc_row(rr)) * D];
    }
    __syncthreads();  // chunk nb's -w, u^T and gates staged
    for (int n = nb; n < n1; ++n) {
      const bool emit = n >= n0;  // the replayed chunk n0 - 1 only rebuilds the state
#pragma unroll
      for (int rt = 0; rt < 8; ++rt) {  // v_new = u, then + (-w) S
        const float4 v = *reinterpret_cast<const float4*>(sU + (16 * jt + acc_col()) * LU + 16 * rt + acc_row(0));
        accV[rt] = f32x4{v.x, v.y, v.z, v.w};
      }
      // S before chunk n into the wave's own columns of sU (just read as u^T there): the loaders
      // store it in the next phase, each thread before it stages the next u^T at those places
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<float4*>(sU + (16 * jt + acc_col()) * LU + 16 * dt + acc_row(0)) =
            make_float4(accS[dt][0], accS[dt][1], accS[dt][2], accS[dt][3]);
      split_product<PS>(accV, ow, accS);
      __syncthreads();  // (k kws)^T of chunk n staged
      const float carry = scarry[n & 1];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) accS[dt] *= carry;
      split_product<PI>(accS, okt, accV, skws[n & 1]);  // S = carry S + k^T (kws v_new)
      if (emit) {
        float* vg = A.vnew + hoff(A, b, h, A.H, n, C, D) + col;
#pragma unroll
        for (int rt = 0; rt < 8; ++rt) st_tile(vg + (size_t)(16 * rt) * D, D, accV[rt]);
      }
      __syncthreads();  // the next chunk's -w, u^T and gates staged
    }
  } else {
    fetch_g(nb);  // prologue: chunk nb's -w, u^T and gates staged, its k in registers
    fetch_k(nb);
    fetch_w(nb);
    fetch_u(nb);
    put_gates(nb);
    put_w();
    put_u();
    __syncthreads();
    for (int n = nb; n < n1; ++n) {
      const int nx = n + 1 < n1 ? n + 1 : n;  // the last step refetches its own chunk (unused)
      put_k();  // k^T of chunk n, for P2 (during P1)
      fetch_g(nx);
      fetch_w(nx);
      fetch_u(nx);
      __syncthreads();
      fetch_k(nx);  // during P2: -w, u^T and the gates of the next chunk
      put_w();
      if (n >= n0) store_s(n);
      put_u();
      if (nx != n) put_gates(nx);  // (the last step's would rewrite the carry being read)
      __syncthreads();
    }
  }
}

// The forward's q strip built from the raw qkv rows of a bf16 I/O conv of 1 to 4 taps at
// C = D = 128 (fuse_q: k_prep skips the q rows), at StripA's layout: lane l holds row
// i0 + l % 16 at channel groups 8 (4s + l / 16) .. + 7. Each lane stages its raw row in LDS, the
// first 48 threads the 3 rows before the chunk (the conv's halo); after a barrier every lane
// reads its lagged rows from there. The conv, SiLU and l2norm run in k_prep's fp32 arithmetic
// and summation order (its 16 lane partials of 8 channels summed pairwise: groups c, c ^ 1
// (lanes l ^ 16), then c ^ 2 (l ^ 32), then within the lane), so the strip holds the values
// k_prep would store. The unit's conv weights go through LDS.
template <int C, int K>
struct RawQ {
  static_assert(C == 128 && K == 128, "the strip of C = D = 128");
  static constexpr int KS = K / 32;
  static constexpr int LDR = 2 * K + 16;        // staged row stride in bytes (16 of padding)
  static constexpr int BYTES = (C + 3) * LDR;   // rows nC - 3 .. nC + C - 1
  Raw8<uint16_t> own[KS], halo;
  float wt;
  __device__ __forceinline__ void fetch(const GdnArgs& A, int b, int hk, int n, int i0) {
    const uint16_t* x = reinterpret_cast<const uint16_t*>(A.qkv);
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3, c0 = hk * K;
#pragma unroll
    for (int s = 0; s < KS; ++s) own[s].load(halo_row<uint16_t>(A, x, b, n * C + i0 + r, c0 + 32 * s + kg));
    const int hi = threadIdx.x < 48 ? threadIdx.x : 0;  // halo row hi / 16, channels 8 (hi % 16) ..
    halo.load(halo_row<uint16_t>(A, x, b, n * C - 3 + hi / 16, c0 + 8 * (hi % 16)));
    const int lag = threadIdx.x / K;  // lags past the taps read lag 0's (a weight of zero when put)
    wt = A.conv_w[(size_t)(lag < A.taps ? A.taps - 1 - lag : A.taps - 1) * A.W + c0 + threadIdx.x % K];
  }
  __device__ __forceinline__ void stage(char* sq, float* sw, const GdnArgs& A, int i0) const {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3;
#pragma unroll
    for (int s = 0; s < KS; ++s) *reinterpret_cast<uint4*>(sq + (i0 + r + 3) * LDR + 2 * (32 * s + kg)) = own[s].a;
    if (threadIdx.x < 48) *reinterpret_cast<uint4*>(sq + (threadIdx.x / 16) * LDR + 16 * (threadIdx.x % 16)) = halo.a;
    sw[threadIdx.x] = (int)threadIdx.x / K < A.taps ? wt : 0.f;
  }
  // after stage and a barrier (the context committed)
  __device__ __forceinline__ void convert(const Ctx<C>& cx, const char* sq, const float* sw, const GdnArgs& A, int n,
                                          int i0, StripA<K>& q) const {
    const int l = lane(), r = l & 15, kg = (l >> 4) << 3, i = i0 + r, t = n * C + i;
    const int st = t < A.T ? cx.seg[i] : 0;
    bool keep[4];
#pragma unroll
    for (int L = 1; L <= 3; ++L) {
      const int j = i - L;
      const int sj = *(j >= 0 ? &cx.seg[j] : &cx.hseg[-1 - j]);
      keep[L] = L < A.taps && (t - L >= 0 || A.init_conv) && sj == st;
    }
    float part[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      float z[8];
#pragma unroll
      for (int L = 0; L <= 3; ++L) {
        Raw8<uint16_t> lr = own[s];  // lag 0: the lane's own row
        if (L > 0) lr.a = *reinterpret_cast<const uint4*>(sq + (i + 3 - L) * LDR + 2 * (32 * s + kg));
        float xl[8];
        lr.get(xl);
        const float4 w0 = *reinterpret_cast<const float4*>(sw + L * K + 32 * s + kg);
        const float4 w1 = *reinterpret_cast<const float4*>(sw + L * K + 32 * s + kg + 4);
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (L == 0) z[e] = xl[e] * w[e];
          else z[e] = keep[L] ? z[e] + xl[e] * w[e] : z[e];
        }
      }
      float sq2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        q.x[s][e] = st > 0 ? z[e] * sigmoid_io<uint16_t>(z[e]) : 0.f;
        sq2 += q.x[s][e] * q.x[s][e];
      }
      part[s] = sq2;
      __builtin_amdgcn_sched_barrier(0);  // one channel group's loads and arithmetic at a time
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {  // k_prep's pairs: groups c ^ 1, then c ^ 2
      part[s] += __shfl_xor(part[s], 16);
      part[s] += __shfl_xor(part[s], 32);
    }
    const float sqs = (part[0] + part[1]) + (part[2] + part[3]);
    float rn = sqs == 0.f ? 0.f : 1.0f / sqrtf(sqs + 1e-6f);
    rn *= A.scale;
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        q.x[s][e] *= rn;
        asm volatile("" : "+v"(q.x[s][e]));  // rounded as k_prep stores it: not fused into the operand split
      }
  }
};

// ---------------------------------------------------------------- k_out
// Persistent: one workgroup per CU (grid <= number of units) loops over the (row, head, chunk)
// units blockIdx.x, + gridDim.x, ...; C/16 waves. Per unit: o = ((q k^T) . D) v_new + q_read
// S_before, token-major output. FQ: q built from the raw rows (RawQ) instead of read from
// k_prep's rows. Every global input of a unit is held in registers and refilled
// with the next unit's values right after it has been used, so its loads run during the rest
// of the unit instead of stalling the next one.
template <int C, int D, int NT, class TS, bool FQ = false>
struct OutIn {
  CtxRaw<C, FQ> cx;
  Regs<C, D, NT> k;      // k rows: B(d, j) = k[j][d]
  std::conditional_t<FQ, RawQ<C, D>, StripA<D>> q;  // this wave's q rows (A operand of q k^T and of q_read S)
  RegsT<C, D, NT> v;     // v_new rows, staged as v_new^T
  RegsT<D, D, NT, true, TS> st;  // S_before rows, staged as S^T
};

template <int C, int D, int PI, int PS, class TIO, bool NORM = false, bool FQ = false>
__global__ __launch_bounds__(C * 4) void k_out(GdnArgs A) {
  constexpr int NT = C * 4;
  constexpr int LI = C + 4;
  constexpr int M = C > D ? C : D;
  using TB = OpTile<PI, M, M>;
  __shared__ __align__(16) float sI[C * LI];  // also the staged raw q rows (FQ)
  __shared__ __align__(16) char sB[TB::BYTES];
  __shared__ Ctx<C> cx;
  __shared__ __align__(16) float snw[NORM ? D : 1];  // the norm's weight
  __shared__ __align__(16) float sWq[FQ ? 4 * D : 4];  // FQ: the unit's conv weights of q
  static_assert(!FQ || (C + 3) * (2 * D + 16) <= C * LI * 4, "FQ: the raw rows staged in sI (RawQ::BYTES)");
  GDN_POISON_LDS(sI, sB, cx, snw, sWq);
  if constexpr (NORM) {
    for (int c = threadIdx.x; c < D; c += NT) snw[c] = A.nw[c];
  }
  const Op<PI> ob = TB::at(sB);
  const int ws = wave_strip<C / 16, false>();
  const int total = A.B * A.H * A.N;
  OutIn<C, D, NT, StateT<PS>, FQ> in;
  {
    const UnitIx<BY_HEAD> x(A, blockIdx.x);
    in.cx.fetch(A, x.b, x.h, x.n);
    in.k.fetch(A.kn + hoff(A, x.b, x.hk, A.Hk, x.n, C, D), D);
    if constexpr (FQ) in.q.fetch(A, x.b, x.hk, x.n, 16 * ws);
    else in.q.fetch(A.qn + hoff(A, x.b, x.hk, A.Hk, x.n, C, D), D, 16 * ws);
    in.v.fetch(A.vnew + hoff(A, x.b, x.h, A.H, x.n, C, D), D);
    in.st.fetch(states_ptr<PS>(A) + ((size_t)x.b * A.H + x.h) * A.N * D * D + (size_t)x.n * D * D, D);
  }
  for (int u = blockIdx.x; u < total; u += gridDim.x) {
    const int w = opaque_uniform(ws), i0 = 16 * w;  // conditions on w stay in the loop
    const UnitIx<BY_HEAD> x(A, u);
    const UnitIx<BY_HEAD> y(A, u + gridDim.x < total ? u + gridDim.x : u);  // the next unit (or this one again)
    in.cx.commit(cx);
    in.cx.fetch(A, y.b, y.h, y.n);
    in.k.put_rows(ob);
    if constexpr (FQ) in.q.stage(reinterpret_cast<char*>(sI), sWq, A, i0);
    __syncthreads();
    derive_ctx<C, NT>(cx);
    StripA<D> qs;  // FQ: the strip built from the staged raw rows
    if constexpr (FQ) in.q.convert(cx, reinterpret_cast<const char*>(sI), sWq, A, x.n, i0, qs);
    else qs = in.q;
    __syncthreads();
    {
      f32x4 acc[C / 16];
      zero(acc);
      qs.template product<PI>(acc, ob, 0, w + 1);
      // refills are issued after the product that follows each staging: the staged
      // registers are then not live across that product
      in.k.fetch(A.kn + hoff(A, y.b, y.hk, A.Hk, y.n, C, D), D);
      const StripDecay<C> sd(cx, i0);
#pragma unroll
      for (int t = 0; t < C / 16; ++t) {
        float d[4];
        sd.tile(cx, i0, t, w, d);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) lds_st(sI + (i0 + acc_row(rr)) * LI + 16 * t + acc_col(), acc[t][rr] * d[rr]);
      }
    }
    __syncthreads();
    in.v.put_cols(ob);
    __syncthreads();
    f32x4 o[D / 16];
    zero(o);
    strip_mma<PI, C, D / 16>(o, krow(sI, LI), i0, ob, 0, 0, tri_end<C>(i0));
    in.v.fetch(A.vnew + hoff(A, y.b, y.h, A.H, y.n, C, D), D);
    __syncthreads();
    in.st.put_cols(ob);
    // the lane's output row after the quad transposes below (4 consecutive columns per tile)
    const int tok = x.n * C + i0 + ((lane() >> 4) << 2) + (lane() & 3);
    const size_t orow = (((size_t)x.b * A.T + (tok < A.T ? tok : 0)) * A.H + x.h) * D + (lane() & 12);
    Raw4<TIO> zr[NORM ? D / 16 : 1];  // the norm's gate, in flight during the last product
    if constexpr (NORM) {
#pragma unroll
      for (int t = 0; t < D / 16; ++t) zr[t].load(reinterpret_cast<const TIO*>(A.nz) + orow + 16 * t);
    }
    __syncthreads();
    qs.template product<PS>(o, ob, 0, D / 16, cx.grow[i0 + (lane() & 15)]);
    if constexpr (FQ) in.q.fetch(A, y.b, y.hk, y.n, i0);
    else in.q.fetch(A.qn + hoff(A, y.b, y.hk, A.Hk, y.n, C, D), D, i0);
    in.st.fetch(states_ptr<PS>(A) + ((size_t)y.b * A.H + y.h) * A.N * D * D + (size_t)y.n * D * D, D);
    TIO* out = reinterpret_cast<TIO*>(A.out);
    {  // quad transposes: each lane stores 4 consecutive columns of one row
      float ss = 0.f;
#pragma unroll
      for (int t = 0; t < D / 16; ++t) {
        float v[4] = {o[t][0], o[t][1], o[t][2], o[t][3]};
        quad_transpose(v);
        if (tok < A.T) st4_io(out + orow + 16 * t, v);
        if constexpr (NORM) {  // the norm reads out as stored
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[t][e] = rnd_io<TIO>(v[e]);
            ss += o[t][e] * o[t][e];
          }
        }
      }
      if constexpr (NORM) {  // gated RMSNorm (norms.py:13-15, 36-40) over the row's 4 lanes
        ss += __shfl_xor(ss, 4);
        ss += __shfl_xor(ss, 8);
        const float r = rsqrt_io<TIO>(ss * (1.0f / D) + A.neps);
        const bool valid = cx.seg[i0 + ((lane() >> 4) << 2) + (lane() & 3)] > 0;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
          float z[4], yv[4];
          zr[t].get(z);
          const float4 w = *reinterpret_cast<const float4*>(snw + 16 * t + (lane() & 12));
          const float wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            yv[e] = valid ? wv[e] * rnd_io<TIO>(o[t][e] * r) * (z[e] * sigmoid_io<TIO>(z[e])) : 0.f;
          if (tok < A.T) st4_io(reinterpret_cast<TIO*>(A.ny) + orow + 16 * t, yv);
        }
      }
    }
    __syncthreads();  // cx and the operand region are rewritten by the next unit
  }
}

// ---------------------------------------------------------------- k_final_state
// grid B*H*(D/DT), 256 threads: the recurrent state after token T-1 of each row, for a decode
// step that continues it (xla.py:141-167 run to the last token). It is the scan's update of
// the last chunk with T-1 as that chunk's last token (the chunk step, pallas_tpu_v2.py:254-269,
// truncated there): S = carry' S_before + sum over the chunk's tokens t <= T-1 of token T-1's
// segment of e^(gamma_{T-1} - gamma_t) k_t v_new_t^T, carry' = e^(gamma_{T-1}) when that
// segment began before the chunk. The rows of v_new up to T-1 do not depend on later rows.
template <int C, int D>
__global__ __launch_bounds__(256) void k_final_state(GdnArgs A) {
  constexpr int DT = D < 32 ? D : 32;
  constexpr int NTL = D / DT;
  constexpr int RG = 256 / DT;              // row groups of a tile
  constexpr int RPT = (D + RG - 1) / RG;    // rows per thread
  __shared__ float sk[C * D];
  __shared__ float sv[C * DT];
  __shared__ float sw[C];
  GDN_POISON_LDS(sk, sv, sw);
  const int tile = blockIdx.x % NTL, bh = blockIdx.x / NTL, h = bh % A.H, b = bh / A.H, hk = h / A.ratio;
  const int last = A.T - 1, nl = last / C, t0 = nl * C, cnt = last - t0 + 1;
  const size_t tb = (size_t)b * A.Tp, th = (size_t)bh * A.Tp;
  const float* kg = A.kn + ((size_t)(b * A.Hk + hk) * A.Tp + t0) * D;
  const float* vg = A.vnew + (th + t0) * D + tile * DT;
  for (int idx = threadIdx.x; idx < cnt * D; idx += 256) sk[idx] = kg[idx];
  for (int idx = threadIdx.x; idx < cnt * DT; idx += 256) sv[idx] = vg[(size_t)(idx / DT) * D + idx % DT];
  const int sl = A.segp[tb + last];
  const float gl = A.gam[th + last], ll = A.gaml[th + last];
  for (int t = threadIdx.x; t < cnt; t += 256)
    sw[t] = A.segp[tb + t0 + t] == sl ? expf((gl - A.gam[th + t0 + t]) + (ll - A.gaml[th + t0 + t])) : 0.f;
  const int before = nl > 0 ? A.segp[tb + t0 - 1] : (A.init_state ? A.segp[tb] : -2);
  const float carry = sl == before ? expf(gl + ll) : 0.f;
  __syncthreads();
  const int j = threadIdx.x % DT, rg = threadIdx.x / DT;
  const float* S = (A.s_last ? A.s_last + (size_t)bh * D * D
                              : static_cast<const float*>(A.states) + ((size_t)bh * A.N + nl) * D * D) + tile * DT + j;
  float acc[RPT];
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg * RPT + r;
    acc[r] = i < D ? carry * S[(size_t)i * D] : 0.f;
  }
  for (int t = 0; t < cnt; ++t) {
    const float wv = sw[t] * sv[t * DT + j];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      const int i = rg * RPT + r;
      if (i < D) acc[r] += sk[t * D + i] * wv;
    }
  }
  float* dst = A.final_state + (size_t)bh * D * D + tile * DT + j;
#pragma unroll
  for (int r = 0; r < RPT; ++r) {
    const int i = rg * RPT + r;
    if (i < D) dst[(size_t)i * D] = acc[r];
  }
}

// ---------------------------------------------------------------- k_conv_state
// grid B, 256 threads: the raw rows T-K+1 .. T-1 of each row (oldest first, [B, K-1, W]), zero
// outside token T-1's segment or before the row's start (there: the given history, if any): the conv history a decode step
// continuing that segment reads (the tap masks of causal_conv1d.py:10-17).
template <class TIO>
__global__ __launch_bounds__(256) void k_conv_state(GdnArgs A) {
  const int b = blockIdx.x, k1 = A.taps - 1, last = A.T - 1;
  const TIO* x = reinterpret_cast<const TIO*>(A.qkv);
  TIO* dst = reinterpret_cast<TIO*>(A.conv_state) + (size_t)b * k1 * A.W;
  const int sl = A.seg[(size_t)b * A.T + last];
  const TIO* hist = reinterpret_cast<const TIO*>(A.init_conv);
  for (long idx = threadIdx.x; idx < (long)k1 * A.W; idx += 256) {  // k1 W can pass 2^31 (W < 2^30)
    const int r = (int)(idx / A.W), c = (int)(idx % A.W), t = last - k1 + 1 + r;
    // rows before the row: the history of a continued sequence (token 0's segment)
    const bool keep = A.seg[(size_t)b * A.T + (t >= 0 ? t : 0)] == sl && (t >= 0 || hist);
    dst[idx] = !keep ? TIO(0) : t >= 0 ? x[((size_t)b * A.T + t) * A.W + c] : hist[((size_t)b * k1 + k1 + t) * A.W + c];
  }
}

// ---------------------------------------------------------------- k_bwd_local
// Persistent over the (row, head, chunk) units as k_out; C/16 waves. Per unit:
// X_loc = T^T (intra^T do) with intra = (q k^T) . D, and Kt = T^T k_write (k_write = kws . k).
// Also stores q k^T's tiles on and below the diagonal (k_bwd_grads' decay pairs read them).
// Every global input is read once per unit into registers: the context, q and k (k for both of
// its stagings: as rows for q k^T, transposed and scaled for k_write^T) are refilled with the
// next unit's values once used; do and T are loaded at the unit's start and after the product
// before their use (holding them longer would spill).
template <int C, int D, int NT, class TIO, class TT>
struct LocalIn {
  CtxRaw<C> cx;
  RegsT<C, D, NT> k;          // k rows
  StripA<D> q;                // this wave's q rows (A operand of q k^T)
  RegsIO<C, D, NT, TIO> dov;  // do rows, staged as do^T
  Regs<C, C, NT, TT> tt;      // T rows (as stored)
  template <class U>
  __device__ __forceinline__ void fetch_k(const GdnArgs& A, const U& y) {
    k.fetch(A.kn + hoff(A, y.b, y.hk, A.Hk, y.n, C, D), D);
  }
  template <class U>
  __device__ __forceinline__ void fetch_q(const GdnArgs& A, const U& y, int i0) {
    q.fetch(A.qn + hoff(A, y.b, y.hk, A.Hk, y.n, C, D), D, i0);
  }
  template <class U>
  __device__ __forceinline__ void fetch_do(const GdnArgs& A, const U& y) {
    const TIO* dout = reinterpret_cast<const TIO*>(A.d_out);
    dov.fetch(dout + (((size_t)y.b * A.T + (size_t)y.n * C) * A.H + y.h) * D, A.H * D, A.T - y.n * C);
  }
  template <class U>
  __device__ __forceinline__ void fetch_t(const GdnArgs& A, const U& y) {
    tt.fetch_lower(static_cast<const TT*>(A.tt) + ((size_t)y.bh * A.N + y.n) * C * C, C);
  }
};

template <int C, int D, int PI, class TIO>
__global__ __launch_bounds__(C * 4) void k_bwd_local(GdnArgs A) {
  constexpr int NT = C * 4;
  constexpr int LA = C + 4;
  constexpr int M = C > D ? C : D;
  using TB = OpTile<PI, M, M>;
  __shared__ float sA[C * LA];
  __shared__ __align__(16) char sB[TB::BYTES];
  __shared__ Ctx<C> cx;
  GDN_POISON_LDS(sA, sB, cx);
  const Op<PI> ob = TB::at(sB);
  const int ws = wave_strip<C / 16, true>();
  const int total = A.B * A.H * A.N;
  LocalIn<C, D, NT, TIO, TinvT<PI>> in;
  {
    const UnitIx<CHUNKS_UP> x(A, blockIdx.x);
    in.cx.fetch(A, x.b, x.h, x.n);
    in.fetch_k(A, x);
    in.fetch_q(A, x, 16 * ws);
  }
  for (int u = blockIdx.x; u < total; u += gridDim.x) {
    const int w = opaque_uniform(ws), i0 = 16 * w;  // conditions on w stay in the loop
    const UnitIx<CHUNKS_UP> x(A, u);
    const UnitIx<CHUNKS_UP> y(A, u + gridDim.x < total ? u + gridDim.x : u);  // the next unit (or this one again)
    in.cx.commit(cx);
    in.cx.fetch(A, y.b, y.h, y.n);
    in.fetch_do(A, x);
    in.k.put_rows(ob);  // B(d, j) = k[j][d]
    __syncthreads();
    derive_ctx<C, NT>(cx);
    __syncthreads();
    {  // intra = (q k^T) . D
      f32x4 acc[C / 16];
      zero(acc);
      in.q.template product<PI>(acc, ob, 0, w + 1);
      in.fetch_q(A, y, i0);
      // q k^T on and below the diagonal, for the decay gradient's pair sums: tile (w, t) as 256
      // floats in accumulator order, one 16-byte piece per lane
      float4* qkg = reinterpret_cast<float4*>(A.qk + (((size_t)x.bh * A.N + x.n) * (C / 16) + w) * (C / 16) * 256);
#pragma unroll
      for (int t = 0; t < C / 16; ++t)
        if (t <= w) qkg[t * 64 + lane()] = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
      const StripDecay<C> sd(cx, i0);
#pragma unroll
      for (int t = 0; t < C / 16; ++t) {
        float d[4];
        sd.tile(cx, i0, t, w, d);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) lds_st(sA + (i0 + acc_row(rr)) * LA + 16 * t + acc_col(), acc[t][rr] * d[rr]);
      }
    }
    __syncthreads();
    constexpr int PDO = exact_b<PI, sizeof(TIO) == 2>();  // do is bf16-exact for bf16 I/O
    in.dov.template put_cols<PI, PDO == P_X3_BEXACT>(ob);
    __syncthreads();
    f32x4 acc[D / 16];
    zero(acc);
    strip_mma<PDO, C, D / 16>(acc, kcol(sA, LA), i0, ob, 0, tri_begin(i0), C);  // dv_loc = intra^T do
    in.fetch_t(A, x);
    __syncthreads();
    in.tt.put_lds_lower(sA, LA);
#pragma unroll
    for (int t = 0; t < D / 16; ++t)  // dv_loc^T: B(c, j) = dv_loc[c][j]
      ob.put4(16 * t + acc_col(), i0 + acc_row(0), acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    __syncthreads();
    zero(acc);
    strip_mma<PI, C, D / 16>(acc, kcol(sA, LA), i0, ob, 0, tri_begin(i0), C);  // T^T dv_loc
    const size_t off = hoff(A, x.b, x.h, A.H, x.n, C, D);
#pragma unroll
    for (int t = 0; t < D / 16; ++t) st_tile(A.xl + off + (size_t)i0 * D + 16 * t, D, acc[t]);
    __syncthreads();
    in.k.put_cols(ob, cx.kws);  // k_write^T
    in.fetch_k(A, y);
    __syncthreads();
    zero(acc);
    strip_mma<PI, C, D / 16>(acc, kcol(sA, LA), i0, ob, 0, tri_begin(i0), C);  // T^T k_write
#pragma unroll
    for (int t = 0; t < D / 16; ++t) st_tile(A.kt + off + (size_t)i0 * D + 16 * t, D, acc[t]);
    __syncthreads();  // cx, T and the operand region are rewritten by the next unit
  }
}

// ---------------------------------------------------------------- k_scan_bwd
// grid B*H*(D/DVT) (XCD-remapped), max(C,D)/16 waves. G [D x DVT] in the accumulators of
// waves < D/16, chunks reversed (pallas_tpu_v2.py:272-291). Also writes, per chunk and tile,
// <G_after, S_before> (d carry, pallas_tpu_v2.py:288). As in the forward scan, every global
// input of a step is held in registers and refilled with the previous chunk's values once used.
template <int C, int D, int DVT, int NT, class TIO>
struct ScanBwdIn {
  PairGates<C> gt;                // wave 0: grow and beta grow of the lane's row pair, and the carry
  AccVals<DVT / 16> sbef;         // S before the chunk, at G's accumulator layout (waves < D/16)
  RegsIO<C, DVT, NT, TIO> dov;    // do columns of the tile, staged as do^T
  StripT<C> qk;                   // the wave's 16 columns of q, staged as (q grow)^T; then of k,
                                  // as (-k beta grow)^T (waves < D/16)
  StripA<D> kt;                   // Kt rows of this wave's strip (waves < C/16)
  AccVals<DVT / 16> xl;           // X_loc at the strip's accumulator layout
  // Loads without branches (a fixed count of memory operations per wave): waves past the
  // D/16 (C/16) strips load a strip they do not use.
  template <int PS>
  __device__ __forceinline__ void fetch_sbef(const GdnArgs& A, int bh, int n, int j0) {
    sbef.fetch(states_ptr<PS>(A) + ((size_t)bh * A.N + n) * D * D + j0, D, 16 * (wave() % (D / 16)));
  }
  __device__ __forceinline__ void fetch_do(const GdnArgs& A, int b, int h, int n, int j0) {
    const TIO* dout = reinterpret_cast<const TIO*>(A.d_out);
    dov.fetch(dout + (((size_t)b * A.T + (size_t)n * C) * A.H + h) * D + j0, A.H * D, A.T - n * C);
  }
  __device__ __forceinline__ void fetch_kt(const GdnArgs& A, int b, int h, int n) {
    kt.fetch(A.kt + hoff(A, b, h, A.H, n, C, D), D, 16 * (wave() % (C / 16)));
  }
  __device__ __forceinline__ void fetch_xl(const GdnArgs& A, int b, int h, int n, int j0) {
    xl.fetch(A.xl + hoff(A, b, h, A.H, n, C, D) + j0, D, 16 * (wave() % (C / 16)));
  }
  __device__ __forceinline__ void fetch_qk(const float* g) { qk.fetch(g, D, 16 * (wave() % (D / 16))); }
  // wave 0: the row scales of the chunk whose gates it holds, into sc[0] (grow), sc[1]
  // (-beta grow) and the carry into sc[2][0]
  __device__ __forceinline__ void put_gates(float (*sc)[C]) const {
    const int j = lane();
    if (j < C / 2) {
      sc[0][2 * j] = gt.grow(0);
      sc[0][2 * j + 1] = gt.grow(1);
      sc[1][2 * j] = -gt.bg(0);
      sc[1][2 * j + 1] = -gt.bg(1);
    }
    if (j == 0) sc[2][0] = gt.carry();
  }
};

template <int C, int D, int DVT, int PI, int PS, class TIO>
__global__ __launch_bounds__((C > D ? C : D) * 4) void k_scan_bwd(GdnArgs A) {
  constexpr int NT = (C > D ? C : D) * 4;
  constexpr int NW = NT / 64;  // wave conditions below are compile-time when every wave takes part
  using TG_ = OpTile<PI, DVT, D>;  // G^T: B(k=dk, j)
  using TQ = OpTile<PI, D, C>;     // (q grow)^T, then (-k beta grow)^T: A(i=dk, k=c)
  using TD = OpTile<PI, DVT, C>;   // do^T and X^T: B(k=c, j)
  __shared__ __align__(16) char sG[TG_::BYTES];
  __shared__ __align__(16) char sQ[TQ::BYTES];
  __shared__ __align__(16) char sDo[TD::BYTES];
  __shared__ __align__(16) char sX[TD::BYTES];
  __shared__ float red[NW];
  __shared__ int red_i[NW];
  __shared__ float sgate[2][3][C];  // per chunk parity: grow, -beta grow, the carry (written by wave 0)
  GDN_POISON_LDS(sG, sQ, sDo, sX, red, red_i, sgate);
  const Op<PI> og = TG_::at(sG), oq = TQ::at(sQ), odo = TD::at(sDo), ox = TD::at(sX);
  const ScanIx ix(A);
  const int tile = ix.tile, bh = ix.bh, part = ix.part;
  const int h = bh % A.H, b = bh / A.H, hk = h / A.ratio;
  const int j0 = tile * DVT;
  const int w = wave();
  // this workgroup's chunks [n0, n1), reversed; from chunk n1 (not stored) when the range ends
  // before the last chunk. That chunk's X is read while the next range may be updating it in
  // place: both values give the same G (its rows that feed G have Kt rows of exact zeros).
  const int n0 = part_start<C, NT, false>(A, b, (int)((long)part * A.N / A.parts), red_i);
  const int n1 = part_start<C, NT, false>(A, b, (int)((long)(part + 1) * A.N / A.parts), red_i);
  if (n0 >= n1) return;
  const int ne = n1 < A.N ? n1 : n1 - 1;
  f32x4 accG[DVT / 16];
  zero(accG);
  if (n1 == A.N && A.d_final && (NW == D / 16 || w < D / 16)) {  // the final state's gradient: G after the last chunk
    const float* g1 = A.d_final + (size_t)bh * D * D + j0;
#pragma unroll
    for (int t = 0; t < DVT / 16; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) accG[t][rr] = g1[(size_t)(16 * w + acc_row(rr)) * D + 16 * t + acc_col()];
  }
  ScanBwdIn<C, D, DVT, NT, TIO> in;
  {
    const int n = ne;
    if (w == 0) {
      in.gt.fetch(A, b, h, n, lane() % (C / 2));
      in.put_gates(sgate[n & 1]);
      in.gt.fetch(A, b, h, n > n0 ? n - 1 : n, lane() % (C / 2));
    }
    in.template fetch_sbef<PS>(A, bh, n, j0);
    in.fetch_do(A, b, h, n, j0);
    in.fetch_qk(A.qn + hoff(A, b, hk, A.Hk, n, C, D));
    in.fetch_kt(A, b, h, n);
    in.fetch_xl(A, b, h, n, j0);
    __syncthreads();
  }
  // Two barriers per step: the q and k operands are staged by each wave into its own rows, and
  // the gates of the next chunk are published by wave 0 between the barriers (two buffers)
  for (int n = ne; n >= n0; --n) {
    const int nx = n > n0 ? n - 1 : n;  // the last step refetches its own chunk (unused)
    const bool emit = n < n1;           // the replayed chunk n1 only rebuilds G
    float part = 0.f;                   // <G after the chunk, S before it> (0 after the last chunk)
    if (NW == D / 16 || w < D / 16) {
      float* gdst = A.gg + ((size_t)bh * A.N + n) * D * D;
#pragma unroll
      for (int t = 0; t < DVT / 16; ++t) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const float g = accG[t][rr];
          og.put(16 * t + acc_col(), 16 * w + acc_row(rr), g);
          part += g * in.sbef.v[t][rr];
        }
        if (emit) st_tile(gdst + 16 * w * D + j0 + 16 * t, D, accG[t]);
      }
      in.template fetch_sbef<PS>(A, bh, nx, j0);
    }
    part = sum64(part);
    if (lane() == 0) red[w] = part;
    const float(*sc)[C] = sgate[n & 1];
    in.dov.template put_cols<PI, exact_b<PI, sizeof(TIO) == 2>() == P_X3_BEXACT>(odo);  // do^T
    in.fetch_do(A, b, h, nx, j0);
    if (NW == D / 16 || w < D / 16) {  // (q grow)^T, the wave's own rows
      in.qk.put(oq, 16 * w, sc[0]);
      in.fetch_qk(A.kn + hoff(A, b, hk, A.Hk, n, C, D));
    }
    __syncthreads();
    if (threadIdx.x == 0 && emit) {
      float s = 0.f;
      for (int q = 0; q < NW; ++q) s += red[q];
      A.gsp[((size_t)bh * A.N + n) * A.ntiles + tile] = s;
    }
    if (NW == C / 16 || w < C / 16) {  // X = X_loc + Kt G
      f32x4 acc[DVT / 16];
      zero(acc);
      in.kt.template product<PS>(acc, og, 0);
      in.fetch_kt(A, b, h, nx);
      const size_t off = hoff(A, b, h, A.H, n, C, D);
#pragma unroll
      for (int t = 0; t < DVT / 16; ++t) {
        f32x4 xv;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          xv[rr] = in.xl.v[t][rr] + acc[t][rr];
          ox.put(16 * t + acc_col(), 16 * w + acc_row(rr), xv[rr]);
        }
        if (emit) st_tile(A.xl + off + (size_t)16 * w * D + j0 + 16 * t, D, xv);
      }
      in.fetch_xl(A, b, h, nx, j0);
    }
    if (NW == D / 16 || w < D / 16) {  // G = carry G + q_read^T do, then (-k beta grow)^T in the same rows
      const float carry = sc[2][0];
#pragma unroll
      for (int t = 0; t < DVT / 16; ++t) accG[t] *= carry;
      strip_mma<exact_b<PI, sizeof(TIO) == 2>(), C, DVT / 16>(accG, oq, 16 * w, odo, 0);  // do: bf16 exact
      in.qk.put(oq, 16 * w, sc[1]);
      in.fetch_qk(A.qn + hoff(A, b, hk, A.Hk, nx, C, D));
    }
    if (w == 0 && nx != n) {  // the next chunk's gates (other buffer: this chunk's are read until the barrier)
      in.put_gates(sgate[nx & 1]);
      in.gt.fetch(A, b, h, nx > n0 ? nx - 1 : nx, lane() % (C / 2));
    }
    __syncthreads();
    if (NW == D / 16 || w < D / 16)  // ... - kbe^T X
      strip_mma<PI, C, DVT / 16>(accG, oq, 16 * w, ox, 0);
    // no barrier here: the next step's writes before its first barrier go to G^T, do^T, the
    // wave's own q rows and red, none of which this product reads
  }
  if (n0 == 0 && A.d_init_state && (NW == D / 16 || w < D / 16)) {  // G before chunk 0: the initial state's gradient
#pragma unroll
    for (int t = 0; t < DVT / 16; ++t) st_tile(A.d_init_state + (size_t)bh * D * D + 16 * w * D + j0 + 16 * t, D, accG[t]);
  }
}

// ---------------------------------------------------------------- k_bwd_grads
// grid B*H*N, C/16 waves. With m1 = strict(-X v_new^T) . D and m2 = (do v_new^T) . D:
//   dkb = m1 k - (grow . X) S^T                    dq  = m2 k + (grow . do) S^T
//   dk' = m1^T (beta k) + m2^T q + (kws . v_new) G^T
//   dk  = dk' + beta dkb    d beta = rows(dkb, k) + rows(X, v)
// (pallas_tpu_v2.py:272-318 regrouped by shared operands; rows(X, v) is added by k_post, which
// rebuilds v). The gradient of the log decays g is emitted as three per-token terms, combined
// by k_post in fp64:
//   dg_t = sum_{s >= t in the chunk} a_s + sum_{s < t} f_s + x_t
//   a = rows(beta k, dkb) + rows(q, (grow do) S^T) - rows(k, m1^T beta k)
//   f = rows(k, (kws v_new) G^T)
//   x_t = sum over token pairs i >= t > j of strict(m2)_ij (q_i . k_j), plus carry <S_before, G_after>
// This is the reference's d gamma (pallas_tpu_v2.py:306-317) reverse-summed over the chunk,
// with terms that cancel in that sum left out: the kws terms (f at its token against their sum
// at the chunk's last), and m2's decay pairs (a pair's row sum against its column sum, summed
// directly over the pairs across t, with q k^T from k_bwd_local). In fp32 those cancelling
// terms leave rounding noise in dg that the sums d A_log = sum dg g amplify; m1's pairs, whose
// noise is an order of magnitude smaller, keep the row-sum form.
// Every input is read from global memory once: each wave holds the X, do and v_new rows of its
// 16-row strip in registers (the A operands of two products each; v_new's rows are also the
// wave's share of the B operand of m1 and m2), and its k and q rows at the accumulator layout
// (its share of the transposed k and q operands, kept for the row sums). Stages: S, v_new, G,
// k^T, q^T through one LDS operand region; m1, then m2, in fp32 LDS (read by rows and by
// columns); the per-token sums through LDS.
template <int C, int D, int PI, int PS, class TIO>
__global__ __launch_bounds__(C * 4) void k_bwd_grads(GdnArgs A) {
  constexpr int NT = C * 4;
  constexpr int LA = C + 4;
  constexpr int M = C > D ? C : D;
  constexpr int TD = D / 16;
  constexpr int TC = C / 16;
  using TB = OpTile<PI, M, M>;
  __shared__ float sA[C * LA];
  __shared__ __align__(16) char sB[TB::BYTES];
  __shared__ Ctx<C> cx;
  __shared__ float sga[C], sgf[C], sgb[C];  // a, f and d beta per token
  __shared__ float sxc[TC * C];             // per wave: its rows' share of x_t for the tokens t of its tiles
  GDN_POISON_LDS(sA, sB, cx, sga, sgf, sgb, sxc);
  const Op<PI> ob = TB::at(sB);
  const int id = blockIdx.x;
  const int n = id % A.N, bh = id / A.N, h = bh % A.H, b = bh / A.H, hk = h / A.ratio;
  const int w = wave_strip<C / 16, true>(), i0 = 16 * w, r = lane() & 15;
  const float* qg = A.qn + hoff(A, b, hk, A.Hk, n, C, D);
  const float* kg = A.kn + hoff(A, b, hk, A.Hk, n, C, D);
  const size_t off = hoff(A, b, h, A.H, n, C, D);
  const TIO* dout = reinterpret_cast<const TIO*>(A.d_out);
  StripA<D> xs, vn;
  StripIO<D, TIO> dos;
  xs.fetch(A.xl + off, D, i0);
  dos.fetch(dout + (((size_t)b * A.T + (size_t)n * C) * A.H + h) * D, A.H * D, i0, A.T - n * C);
  load_ctx<C, NT>(cx, A, b, h, n);
  stage_rows<D, D, NT>(ob, states_ptr<PS>(A) + ((size_t)bh * A.N + n) * D * D, D);  // S: B(dv, j=dk) = S[dk][dv]
  vn.fetch(A.vnew + off, D, i0);
  __syncthreads();
  f32x4 dkb[TD], dq[TD];
  zero(dkb);
  zero(dq);
  xs.template product<PS>(dkb, ob, 0, TD, -cx.grow[i0 + r]);  // -(grow X) S^T
  dos.template product<PS>(dq, ob, 0, TD, cx.grow[i0 + r]);   // (grow do) S^T
  __syncthreads();
  vn.put_rows(ob, i0);  // v_new: B(dv, j) = v_new[j][dv]
  __syncthreads();
  f32x4 m2[TC];
  {  // m1 -> LDS, m2 -> registers
    f32x4 acc[TC];
    zero(acc);
    const StripDecay<C> sd(cx, i0);
    xs.template product<PI>(acc, ob, 0, w + 1);
    float dn[4];  // the next tile's decays, read before this tile's stores (their memory clobber)
    sd.tile(cx, i0, 0, w, dn);
#pragma unroll
    for (int t = 0; t < TC; ++t) {
      const float d[4] = {dn[0], dn[1], dn[2], dn[3]};
      if (t + 1 < TC) sd.tile(cx, i0, t + 1, w, dn);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int i = i0 + acc_row(rr), j = 16 * t + acc_col();
        lds_st(sA + i * LA + j, i > j ? -acc[t][rr] * d[rr] : 0.f);
      }
    }
    AccVals<TC> qk;  // q k^T of the strip from k_bwd_local (tiles past the diagonal: the diagonal again)
    {
      const float4* g = reinterpret_cast<const float4*>(A.qk + (((size_t)bh * A.N + n) * TC + w) * TC * 256);
#pragma unroll
      for (int t = 0; t < TC; ++t) {
        const float4 v = g[(t < w ? t : w) * 64 + lane()];
        qk.v[t][0] = v.x;
        qk.v[t][1] = v.y;
        qk.v[t][2] = v.z;
        qk.v[t][3] = v.w;
      }
    }
    zero(m2);
    dos.template product<exact_a<PI, sizeof(TIO) == 2>()>(m2, ob, 0, w + 1);  // do: bf16 exact
    float rp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < TC; ++t) {
      float d[4];
      sd.tile(cx, i0, t, w, d);
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) m2[t][rr] *= d[rr];
      if (t <= w) {  // x's pairs: strict(m2) . (q k^T)
        f32x4 e;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) e[rr] = (t < w || acc_row(rr) > acc_col()) ? m2[t][rr] * qk.v[t][rr] : 0.f;
        float cp = 0.f;
        cross_tile(e, t == w, rp, cp);
        if (lane() < 16) sxc[w * C + 16 * t + lane()] = cp;
      }
    }
  }
  __syncthreads();
  stage_rows<D, D, NT>(ob, A.gg + ((size_t)bh * A.N + n) * D * D, D);  // G
  __syncthreads();
  f32x4 dk[TD];
  zero(dk);
  vn.template product<PS>(dk, ob, 0, TD, cx.kws[i0 + r]);  // (kws v_new) G^T
  AccVals<TD> kk;  // (k and q are fetched late: live across the stages before, they would spill)
  kk.fetch(kg, D, i0);
  __syncthreads();
#pragma unroll
  for (int t = 0; t < TD; ++t)  // k^T: B(c, j) = k[c][j]
    ob.put4(16 * t + acc_col(), i0 + acc_row(0), kk.v[t][0], kk.v[t][1], kk.v[t][2], kk.v[t][3]);
  {  // f = rows(k, (kws v_new) G^T), before m1^T beta k joins dk' (per token, in LDS)
    float rf[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < TD; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) rf[rr] += kk.v[t][rr] * dk[t][rr];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      rf[rr] = sum16(rf[rr]);
      if (acc_col() == 0) sgf[i0 + acc_row(rr)] = rf[rr];
    }
  }
  __syncthreads();
  strip_mma<PI, C, TD>(dkb, krow(sA, LA), i0, ob, 0, 0, tri_end<C>(i0));                  // m1 k
  strip_mma<PI, C, TD>(dk, scale_k(kcol(sA, LA), cx.beta), i0, ob, 0, tri_begin(i0), C);  // m1^T beta k
  // dkb is complete: its row sums with k (d beta) and those of dk' so far, then dkb folded
  // into dk. a = rows(beta k, dkb) + rows(q, (grow do) S^T) - rows(k, m1^T beta k): the
  // e^gamma terms and m1's decay pairs (pallas_tpu_v2.py:306-310) as row sums
  {
    float r4[4] = {0.f, 0.f, 0.f, 0.f}, r3[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < TD; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        r4[rr] += dkb[t][rr] * kk.v[t][rr];
        r3[rr] += kk.v[t][rr] * dk[t][rr];
        dk[t][rr] += cx.beta[i0 + acc_row(rr)] * dkb[t][rr];
      }
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      r4[rr] = sum16(r4[rr]);
      r3[rr] = sum16(r3[rr]);
      const int i = i0 + acc_row(rr);
      if (acc_col() == 0) {
        sgb[i] = r4[rr];
        sga[i] = cx.beta[i] * r4[rr] - (r3[rr] - sgf[i]);
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int t = 0; t < TC; ++t)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) lds_st(sA + (i0 + acc_row(rr)) * LA + 16 * t + acc_col(), m2[t][rr]);
  AccVals<TD> qq;
  qq.fetch(qg, D, i0);
  __syncthreads();
  {  // a's rows(q, (grow do) S^T), before m2 k joins dq
    float ra[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < TD; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) ra[rr] += qq.v[t][rr] * dq[t][rr];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      ra[rr] = sum16(ra[rr]);
      if (acc_col() == 0) sga[i0 + acc_row(rr)] += ra[rr];
    }
  }
  strip_mma<PI, C, TD>(dq, krow(sA, LA), i0, ob, 0, 0, tri_end<C>(i0));  // m2 k
  __syncthreads();
#pragma unroll
  for (int t = 0; t < TD; ++t)  // q^T
    ob.put4(16 * t + acc_col(), i0 + acc_row(0), qq.v[t][0], qq.v[t][1], qq.v[t][2], qq.v[t][3]);
  __syncthreads();
  f32x4 dk2[TD];
  zero(dk2);
  strip_mma<PI, C, TD>(dk2, kcol(sA, LA), i0, ob, 0, tri_begin(i0), C);  // m2^T q
  // epilogue: the per-value-head dq, dk and the per-token gate terms
#pragma unroll
  for (int t = 0; t < TD; ++t)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int i = i0 + acc_row(rr), j = 16 * t + acc_col();
      A.dqh[off + i * D + j] = dq[t][rr];
      A.dkh[off + i * D + j] = dk[t][rr] + dk2[t][rr];
    }
  const size_t tok = (size_t)bh * A.Tp + (size_t)n * C;
  if (threadIdx.x < C) {  // the per-token terms; x_t: the waves' pair sums and the carry term
    const int t = threadIdx.x;
    float x = 0.f, dcarry = 0.f;
    for (int v = t / 16; v < TC; ++v) x += sxc[v * C + t];
    for (int q = 0; q < A.ntiles; ++q) dcarry += A.gsp[((size_t)bh * A.N + n) * A.ntiles + q];
    A.dgam[tok + t] = sga[t];
    A.dkws[tok + t] = sgf[t];
    A.dbet[tok + t] = sgb[t];
    A.dcross[tok + t] = x + cx.carry * dcarry;
  }
}

// ---------------------------------------------------------------- k_post
// grid B*N*(2*Hk + H) as k_prep's, 256 threads: the activations' gradients back to d(qkv) -- GQA sums,
// l2norm backward (pallas_tpu_mega.py:101-103), SiLU and the anti-causal conv backward with
// segment masks (pallas_tpu_mega.py:161-179, 306-319) -- and, for the value heads, the gate
// backward (pallas_tpu_mega.py:129-145): dg = reverse in-chunk cumsum of d gamma, and d beta
// completed with rows(X, v) from the rebuilt v. DW: also this chunk's partial of d(conv w)
// (pallas_tpu_mega.py:527-535), launched only when it is wanted.
template <int C, int D, class TIO, class TG, int HW, bool DW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_post(GdnArgs A) {
  static_assert(HW == 3 || HW == 4, "the conv halo: taps - 1 rows (launched with HW >= taps - 1)");
  constexpr int CG = D / 8;
  constexpr int NG = 256 / CG;                  // row groups of CG lanes
  constexpr int RG = (C + HW + NG - 1) / NG;    // consecutive rows per group: the chunk's, then HW look-ahead rows
  constexpr int HS = RG < HW ? RG : HW;         // a group's first rows, read by the groups before it
  constexpr int LZ = D + 4;
  constexpr int NL = HW + 1;                    // lags 0 .. taps - 1
  __shared__ float shd[NG * HS * LZ];           // dz of each group's first HS rows
  __shared__ int shs[NG * HS];                  // and their segment ids
  __shared__ float sxv[C];                      // value heads: rows(X, v) of the chunk's tokens
  __shared__ float sdw[DW ? 4 * NL * D : 1];    // per-wave sums of d(conv w)
  GDN_POISON_LDS(shd, shs, sxv, sdw);
  const int slots = 2 * A.Hk + A.H, bn = blockIdx.x / slots;
  const int b = bn / A.N, n = bn % A.N;
  const int slot = blockIdx.x % slots;
  const int cg = threadIdx.x % CG, grp = threadIdx.x / CG;
  int kind, head, c0;
  if (slot < A.Hk) { kind = 0; head = slot; c0 = slot * D; }
  else if (slot < 2 * A.Hk) { kind = 1; head = slot - A.Hk; c0 = A.Hk * D + head * D; }
  else { kind = 2; head = slot - 2 * A.Hk; c0 = 2 * A.Hk * D + head * D; }
  const int cc = c0 + cg * 8;
  const int taps = A.taps;
  const TIO* x = reinterpret_cast<const TIO*>(A.qkv);
  TIO* dx = reinterpret_cast<TIO*>(A.d_qkv);
  const int32_t* sp = A.segp + (size_t)b * A.Tp;
  // the gate backward's inputs (value heads, wave 0), fetched first so that they arrive
  // during the chunk's rows
  constexpr int E = (C + 63) / 64;
  const bool gate_wave = kind == 2 && threadIdx.x < 64;
  const size_t tok = (size_t)(b * A.H + head) * A.Tp + (size_t)n * C;
  float gdg[E], gdk[E], gdx[E], gdb[E], gav[E], gbv[E];
  if (gate_wave) {
    const TG* ga = reinterpret_cast<const TG*>(A.ga);
    const TG* gb = reinterpret_cast<const TG*>(A.gb);
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int i = threadIdx.x * E + q, t = n * C + i;
      const int ic = i < C ? i : C - 1, tc = t < A.T ? t : A.T - 1;
      gdg[q] = A.dgam[tok + ic];
      gdk[q] = A.dkws[tok + ic];
      gdx[q] = A.dcross[tok + ic];
      gdb[q] = A.dbet[tok + ic];
      gav[q] = ldf(ga + ((size_t)b * A.T + tc) * A.H + head);
      gbv[q] = ldf(gb + ((size_t)b * A.T + tc) * A.H + head);
    }
  }
  float wl[5][8];
  lag_weights(A, cc, wl);
  const int rows = C + (taps > 1 ? taps - 1 : 0);
  // Each group owns RG consecutive rows: their raw rows with the conv halo, segment ids and
  // incoming gradients are all loaded first (clamped addresses, no branches), then dz row by
  // row from registers; dx of a row follows as soon as dz of its HW look-ahead rows is there,
  // and the last HW rows take the next groups' first rows from LDS after one barrier.
  const int r0 = grp * RG;
  Raw8<TIO> raw[RG + HW];
  int sgv[RG + HW];
#pragma unroll
  for (int i = 0; i < RG + HW; ++i) {
    const int tt = n * C + r0 - HW + i;
    const int ts = tt < 0 ? 0 : (tt < A.Tp ? tt : A.Tp - 1);
    raw[i].load(halo_row<TIO>(A, x, b, tt, cc));
    sgv[i] = sp[ts];  // rows before the row: token 0's segment (the history of a continued sequence)
  }
  float dyv[RG][8], btv[RG];
#pragma unroll
  for (int i = 0; i < RG; ++i) {
    const int t = n * C + r0 + i, tl = t < A.Tp ? t : A.Tp - 1;
    if (kind < 2) {  // GQA sum over the value heads of this key head
      const float* src = (kind == 0 ? A.dqh : A.dkh) + ((size_t)(b * A.H + head * A.ratio) * A.Tp + tl) * D + cg * 8;
      ld8(src, dyv[i]);
      for (int v = 1; v < A.ratio; ++v) {
        float y[8];
        ld8(src + (size_t)v * A.Tp * D, y);
#pragma unroll
        for (int e = 0; e < 8; ++e) dyv[i][e] += y[e];
      }
    } else {  // dv = X beta
      ld8(A.xl + ((size_t)(b * A.H + head) * A.Tp + tl) * D + cg * 8, dyv[i]);
      btv[i] = A.bet[(size_t)(b * A.H + head) * A.Tp + tl];
    }
  }
  float dzr[RG][8];
  int str[RG];
  // dx of own row j (rows < C of real tokens): the anti-causal conv,
  // dx[t] = sum over lags of w[K-1-L] keep_L[t+L] dz[t+L]; `ext` rows come from LDS
  auto emit = [&](int j, bool ext) {
    const int r = r0 + j, t = n * C + r;
    if (r >= C || t >= A.T) return;
    float o[8];
    if (taps == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = dzr[j][e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = dzr[j][e] * wl[0][e];
#pragma unroll
      for (int L = 1; L <= HW; ++L) {
        if (j + L < RG) {
          if (L < taps && str[j + L] == str[j]) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += wl[L][e] * dzr[j + L][e];
          }
        } else if (ext) {  // row r + L: the first rows of group grp + (j + L) / RG (r + L < C + HW)
          const int k = (grp + (j + L) / RG) * HS + (j + L) % RG;
          if (L < taps && shs[k] == str[j]) {
            const float4* q = reinterpret_cast<const float4*>(shd + k * LZ + cg * 8);
            const float4 p0 = q[0], p1 = q[1];
            o[0] += wl[L][0] * p0.x; o[1] += wl[L][1] * p0.y; o[2] += wl[L][2] * p0.z; o[3] += wl[L][3] * p0.w;
            o[4] += wl[L][4] * p1.x; o[5] += wl[L][5] * p1.y; o[6] += wl[L][6] * p1.z; o[7] += wl[L][7] * p1.w;
          }
        }
      }
    }
    st8_io_nt(dx + ((size_t)b * A.T + t) * A.W + cc, o);  // d(qkv): read by no later kernel
  };
#pragma unroll
  for (int i = 0; i < RG; ++i) {
    const int r = r0 + i, t = n * C + r;
    const bool live = r < rows && t < A.Tp;  // uniform over the CG lanes of the row
    const int st = live ? sgv[HW + i] : -3;
    float z[8], sg[8], act[8], dy[8];
    if (taps == 0) {
      raw[HW + i].get(act);
#pragma unroll
      for (int e = 0; e < 8; ++e) act[e] = t < A.T ? act[e] : 0.f;
    } else {  // z = sum over lags of keep * x[t-L] * w[K-1-L], lag 0 first
      raw[HW + i].get(z);
#pragma unroll
      for (int e = 0; e < 8; ++e) z[e] *= wl[0][e];
#pragma unroll
      for (int L = 1; L <= HW; ++L) {
        const bool keep = L < taps && (t - L >= 0 || A.init_conv) && sgv[HW + i - L] == st;
        float xl[8];
        raw[HW + i - L].get(xl);
#pragma unroll
        for (int e = 0; e < 8; ++e) z[e] = keep ? z[e] + xl[e] * wl[L][e] : z[e];
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        sg[e] = sigmoid_io<TIO>(z[e]);  // once: SiLU and its backward
        act[e] = st > 0 ? z[e] * sg[e] : 0.f;
      }
    }
    if (kind < 2) {  // l2norm backward (q's scale first)
#pragma unroll
      for (int e = 0; e < 8; ++e) dy[e] = kind == 0 ? dyv[i][e] * A.scale : dyv[i][e];
      float sq = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) sq += act[e] * act[e];
      sq = sum_lanes<CG>(sq);
      const float rn = sq == 0.f ? 0.f : 1.0f / sqrtf(sq + 1e-6f);
      float dot = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) dot += act[e] * rn * dy[e];
      dot = sum_lanes<CG>(dot);
#pragma unroll
      for (int e = 0; e < 8; ++e) dy[e] = rn * (dy[e] - act[e] * rn * dot);
    } else {  // dv = X beta, and rows(X, v) for d beta (v is this head's activation)
      float xv = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dy[e] = dyv[i][e] * btv[i];
        xv += dyv[i][e] * act[e];
      }
      xv = sum_lanes<CG>(xv);
      if (cg == 0 && r < C) sxv[r] = xv;
    }
    if (taps == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e) dzr[i][e] = live ? dy[e] : 0.f;
    } else {  // SiLU backward on valid tokens
#pragma unroll
      for (int e = 0; e < 8; ++e) dzr[i][e] = (live && st > 0) ? dy[e] * sg[e] * (1.f + z[e] * (1.f - sg[e])) : 0.f;
    }
    str[i] = st;
    if (i < HS) {
      float4* o = reinterpret_cast<float4*>(shd + (grp * HS + i) * LZ + cg * 8);
      o[0] = make_float4(dzr[i][0], dzr[i][1], dzr[i][2], dzr[i][3]);
      o[1] = make_float4(dzr[i][4], dzr[i][5], dzr[i][6], dzr[i][7]);
      if (cg == 0) shs[grp * HS + i] = st;
    }
    if (i >= HW) emit(i - HW, false);
  }
  __syncthreads();
#pragma unroll
  for (int j = (RG > HW ? RG - HW : 0); j < RG; ++j) emit(j, true);
  if (n == 0 && grp == 0 && A.d_init_conv && taps > 1) {
    // the gradient of the history rows -p (p = 1 .. taps - 1): sum over lags L >= p of
    // w[K-1-L] dz[L - p] on rows of token 0's segment (rows past the group's from LDS)
    const int s0 = sp[0];
#pragma unroll
    for (int p = 1; p <= HW; ++p) {
      if (p >= taps) break;
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int L = p; L <= HW; ++L) {
        if (L >= taps) break;
        const int j = L - p;
        if (j < RG) {
          if (str[j] == s0) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += wl[L][e] * dzr[j][e];
          }
        } else {
          const int k = (j / RG) * HS + j % RG;
          if (shs[k] == s0) {
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] += wl[L][e] * shd[k * LZ + cg * 8 + e];
          }
        }
      }
      st8_io(reinterpret_cast<TIO*>(A.d_init_conv) + ((size_t)b * (taps - 1) + (taps - 1 - p)) * A.W + cc, o);
    }
  }
  if constexpr (DW) {
    // d w[K-1-L] += keep_L[t] dz[t] x[t-L] over the group's rows of the chunk, from its raw rows
    // loaded again (cache hits) once the prefetched gradients are spent
    float dwa[NL][8];
#pragma unroll
    for (int L = 0; L < NL; ++L)
#pragma unroll
      for (int e = 0; e < 8; ++e) dwa[L][e] = 0.f;
#pragma unroll
    for (int i = 0; i < RG + HW; ++i) raw[i].load(halo_row<TIO>(A, x, b, n * C + r0 - HW + i, cc));
#pragma unroll
    for (int i = 0; i < RG; ++i) {
      const int r = r0 + i, t = n * C + r;
#pragma unroll
      for (int L = 0; L < NL; ++L) {
        const bool keep = r < C && L < taps && (t - L >= 0 || A.init_conv) && (L == 0 || sgv[HW + i - L] == str[i]);
        float xl[8];
        raw[HW + i - L].get(xl);
#pragma unroll
        for (int e = 0; e < 8; ++e) dwa[L][e] = keep ? dwa[L][e] + dzr[i][e] * xl[e] : dwa[L][e];
      }
    }
    // this chunk's partial: the wave's groups summed by shuffles, then the waves, fixed order
#pragma unroll
    for (int L = 0; L < NL; ++L)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float v = dwa[L][e];
#pragma unroll
        for (int m = CG; m < 64; m <<= 1) v += __shfl_xor(v, m);
        if (lane() < CG) sdw[(wave() * NL + L) * D + cg * 8 + e] = v;
      }
    __syncthreads();
    for (int idx = threadIdx.x; idx < taps * D; idx += 256) {
      const int L = idx / D, c = idx % D;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) s += sdw[(w * NL + L) * D + c];
      A.dwp[(((size_t)b * A.N + n) * taps + (taps - 1 - L)) * A.W + c0 + c] = s;
    }
  }
  if (gate_wave) {  // gate backward of value head `head`
    const int l = threadIdx.x;
    TG* da = reinterpret_cast<TG*>(A.d_a);
    TG* db = reinterpret_cast<TG*>(A.d_b);
    const float ea = expf(A.a_log[head]), dtb = A.dt_bias[head];
    // dg from its three per-token terms, and the A_log / dt_bias partial sums, in fp64
    double dgv[E];
    chunk_dg<C, E>(gdg, gdk, gdx, dgv);
    double sa = 0.0, sd = 0.0;
#pragma unroll
    for (int q = 0; q < E; ++q) {
      const int i = l * E + q, t = n * C + i;
      if (i < C) {
        const bool in = t < A.T;
        const float av = in ? gav[q] : 0.f;
        const float bv = in ? gbv[q] : 0.f;
        const double dg = dgv[q];
        const float xg = av + dtb;
        const float g = -ea * softplusf_(xg);
        const double dad = dg * (double)(-ea * sigmoidf_(xg));
        const float dav = (float)dad;
        const float bt = sigmoidf_(bv);
        const float dbv = (gdb[q] + sxv[i]) * bt * (1.f - bt);
        // the padded tail's g is the constant 0 (no function of A_log, dt_bias): its dg, which the
        // final state's gradient makes nonzero, enters neither sum
        sa += in ? dg * (double)g : 0.0;
        sd += in ? dad : 0.0;
        if (in) {
          stf(da + ((size_t)b * A.T + t) * A.H + head, dav);
          stf(db + ((size_t)b * A.T + t) * A.H + head, dbv);
        }
      }
    }
    sa = sum64d(sa);
    sd = sum64d(sd);
    if (l == 0) {
      A.pa[((size_t)b * A.N + n) * A.H + head] = sa;
      A.pd[((size_t)b * A.N + n) * A.H + head] = sd;
    }
  }
}

// ---------------------------------------------------------------- k_reduce
// d A_log[h] = sum over rows and chunks of the per-chunk partials, likewise d dt_bias and
// the conv weight (pallas_tpu_mega.py:527-535, 563-568); fixed order, no atomics. Workgroups
// 0..H-1: one value head each, the partials summed by 256 threads in fp64 then by a fixed
// tree; the rest: one conv weight per thread.
template <int C>
__global__ __launch_bounds__(256) void k_reduce(GdnArgs A) {
  const int bn = A.B * A.N;
  if ((int)blockIdx.x < A.H) {
    __shared__ double ra[256], rd[256];
    GDN_POISON_LDS(ra, rd);
    const int h = blockIdx.x;
    double sa = 0.0, sd = 0.0;
    for (int q = threadIdx.x; q < bn; q += 256) {
      sa += A.pa[(size_t)q * A.H + h];
      sd += A.pd[(size_t)q * A.H + h];
    }
    ra[threadIdx.x] = sa;
    rd[threadIdx.x] = sd;
    __syncthreads();
    for (int m = 128; m > 0; m >>= 1) {
      if ((int)threadIdx.x < m) {
        ra[threadIdx.x] += ra[threadIdx.x + m];
        rd[threadIdx.x] += rd[threadIdx.x + m];
      }
      __syncthreads();
    }
    if (threadIdx.x == 0) {
      A.d_a_log[h] = (float)ra[0];
      A.d_dt_bias[h] = (float)rd[0];
    }
  } else {
    const int j = ((int)blockIdx.x - A.H) * 256 + threadIdx.x;
    if (A.d_conv_w && A.taps > 0 && j < A.taps * A.W) {
      float s = 0.f;
      for (int q = 0; q < bn; ++q) s += A.dwp[(size_t)q * A.taps * A.W + j];
      A.d_conv_w[j] = s;
    }
  }
}

}  // namespace gdn
