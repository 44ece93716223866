// Kernel arguments of the GDN kernel sequences: shapes, tensors and workspace slices.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace gdn {

struct GdnArgs {
  int B, T, Tp, N, Hk, H, ratio, taps, W;
  int ntiles;  // Dv tiles of the scans
  int parts;   // chunk ranges per (row, head, tile) of the scans, split where a segment resets
  int res;     // residuals kept by the forward: 0 states, 1 and T, 2 and v_new
  int inv;     // the in-chunk inverse: 0 pure doubling, 1 diagonal blocks by substitution + doubling
  int fuse_q;  // the forward's k_out builds q from the raw rows, k_prep skips them (k_out's RawQ)
  int fuse_v;  // the forward's k_chunk builds v from the raw rows, k_prep skips them (k_chunk's RawV);
               // the caller's fuse_v allows both, the launch sequence decides each (the
               // forward's workspace then has no fp32 rows of what is built)
  float scale; // Dk^-1/2
  // inputs
  const void* qkv;
  const void* ga;
  const void* gb;
  const float* a_log;
  const float* dt_bias;
  const float* conv_w;
  const int32_t* seg;
  // forward outputs
  void* out;
  // the gated RMSNorm of out computed in the output kernel (null ny: none): y = w rnd(x r) silu(z)
  // with x = out as stored, r = rsqrt(mean x^2 + eps), 0 on padding tokens
  const void* nz;    // [B, T, H, Dv] io dtype, the gate
  const float* nw;   // [Dv]
  float neps;
  void* ny;          // [B, T, H, Dv] io dtype
  void* states;        // [B, H, N, Dk, Dv] fp32, or bf16 when the state-path products are one bf16
                       // pass (precisions mixed and bf16: StateT in gdn_kernels.h)
  float* s_last;       // [B, H, Dk, Dv] fp32 copy of the state before the last chunk when the
                       // states are bf16 (k_final_state reads it), else null
  float* final_state;  // [B, H, Dk, Dv] the state after token T-1 (or null)
  void* conv_state;    // [B, K-1, W] the raw rows before token T (or null)
  // a sequence continued from an earlier call: the state before token 0 (chunk 0's tokens of
  // token 0's segment read it) and the K-1 raw rows before token 0 (token 0's segment); null:
  // a fresh start (state 0, chunk 0 reads nothing; no rows before the row)
  const float* init_state;  // [B, H, Dk, Dv]
  const void* init_conv;    // [B, K-1, W] io dtype
  const float* d_final;     // [B, H, Dk, Dv] the gradient of final_state (or null: 0)
  float* d_init_state;      // [B, H, Dk, Dv] (or null)
  void* d_init_conv;        // [B, K-1, W] io dtype (or null)
  // the v2 operator's inputs q, k [B,T,Hk,D], v [B,T,H,D], g, beta [B,T,H] and their gradients
  const void* q2;
  const void* k2;
  const void* v2;
  const void* g2;
  const void* b2;
  void* d_q2;
  void* d_k2;
  void* d_v2;
  void* d_g2;
  void* d_b2;
  // backward
  const void* d_out;
  void* d_qkv;
  void* d_a;
  void* d_b;
  float* d_a_log;
  float* d_dt_bias;
  float* d_conv_w;
  // workspace
  int32_t* segp;  // [B, Tp]
  float* qn;      // [B, Hk, Tp, D]  l2norm(q) * Dk^-1/2
  float* kn;      // [B, Hk, Tp, D]  l2norm(k)
  float* vv;      // [B, H, Tp, D]   post-conv v
  float* gam;     // [B, H, Tp]      in-chunk cumulative log decay (fp32 high part)
  float* gaml;    // [B, H, Tp]      its low part: gamma = gam + gaml to fp64 accuracy
  float* bet;     // [B, H, Tp]      beta
  float* uu;      // [B, H, Tp, D]   u = T v beta            (forward)
  float* ww;      // [B, H, Tp, D]   w = T kbe               (forward)
  float* vnew;    // [B, H, Tp, D]   v_new
  void* tt;       // [B, H, N, C, C] T = (I+L)^-1, fp32 (bf16 under precision bf16) (backward: only the 16 x 16 tiles on and
                  // below the diagonal are written and read)
  float* qk;      // [B, H, N, C/16, C/16, 256] q k^T's 16 x 16 tiles on and below the diagonal, in
                  // accumulator order (backward)
  float* xl;      // [B, H, Tp, D]   X_loc, then X
  float* kt;      // [B, H, Tp, D]   T^T k_write
  float* gg;      // [B, H, N, D, D] G after each chunk
  float* gsp;     // [B, H, N, ntiles] <G_after, S_before> per Dv tile (d carry)
  float* dqh;     // [B, H, Tp, D]   dq per value head
  float* dkh;     // [B, H, Tp, D]   dk per value head
  float* dgam;    // [B, H, Tp]      d g terms summed over the chunk's later tokens (e^gamma factors)
  float* dkws;    // [B, H, Tp]      d g terms summed over the chunk's earlier tokens (e^(gamma_C - gamma))
  float* dcross;  // [B, H, Tp]      d g terms of the token itself (decay pairs across it, the carry)
  float* dbet;    // [B, H, Tp]
  double* pa;     // [B, N, H] partial d A_log (fp64)
  double* pd;     // [B, N, H] partial d dt_bias (fp64)
  float* dwp;     // [B*N, K, W] partial d conv weight (or null)
};

}  // namespace gdn
