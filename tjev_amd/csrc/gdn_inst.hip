// One (chunk, head dim) instantiation of the kernel sequences, built once per GDN_SHAPE in
// gdn_shapes.def with -DGDN_C=<chunk> -DGDN_D=<head dim>, in six object files
// (-DGDN_PART=0 .. 5): part 0 holds the launch sequences, the shape's table and the small
// kernels; parts 1 .. 5 each instantiate one family of the large kernels (explicit
// instantiations, declared extern in the other parts). A kernel's code then depends only on its
// own family's source: the register allocation of one family, which runs close to the 256
// VGPRs of two waves per SIMD, no longer moves when another family's code changes.
#ifndef GDN_PART
#error "build with -DGDN_PART=<part> (0 .. 5)"
#endif
// 32-bit lane offsets in the staging loads of the scans, k_out and k_bwd_local (measured:
// k_bwd_local 222 -> 200 us, the others 2 us each); k_chunk and k_bwd_grads keep the widened
// form (with 32-bit offsets they spill: +7 and +35 us)
#if GDN_PART == 2 || GDN_PART == 3 || GDN_PART == 4
#define GDN_LANE_OFF32 1
#endif
#include "gdn_kernels.h"
#include "gdn_launch.h"
#include "gdn_v2.h"

#ifndef GDN_C
#error "build with -DGDN_C=<chunk> -DGDN_D=<head dim> -DGDN_PART=<part>"
#endif

namespace gdn {

// the explicit instantiations of parts 1 .. 5 (definitions in their own part, declarations
// elsewhere), over every (A-side, state-side) precision pair the shape table holds
#if GDN_PART == 1
#define GDN_KW_1 template
#else
#define GDN_KW_1 extern template
#endif
#if GDN_PART == 2
#define GDN_KW_2 template
#else
#define GDN_KW_2 extern template
#endif
#if GDN_PART == 3
#define GDN_KW_3 template
#else
#define GDN_KW_3 extern template
#endif
#if GDN_PART == 4
#define GDN_KW_4 template
#else
#define GDN_KW_4 extern template
#endif
#if GDN_PART == 5
#define GDN_KW_5 template
#else
#define GDN_KW_5 extern template
#endif
constexpr int kDVT = GDN_D < 32 ? GDN_D : 32;
#define GDN_EACH_PAIR(M) M(P_F32, P_F32) M(P_BF16X3, P_BF16X3) M(P_BF16, P_BF16) M(P_BF16X3, P_BF16)
#define GDN_EACH_IO(M, PI, PS) M(PI, PS, float) M(PI, PS, uint16_t)
// part 1: k_chunk, its four modes (the three that invert with either form of the inverse)
#define GDN_CHUNK_INV(PI, PS, DBL)                                             \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 0, DBL>(GdnArgs);     \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 1, DBL>(GdnArgs);     \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 2, DBL>(GdnArgs);
#define GDN_CHUNK(PI, PS)          \
  GDN_CHUNK_INV(PI, PS, true)      \
  GDN_CHUNK_INV(PI, PS, false)     \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 3, false>(GdnArgs);
GDN_EACH_PAIR(GDN_CHUNK)
#if GDN_C == 128 && GDN_D == 128  // and the forward's with v from the raw rows (bf16 I/O)
#define GDN_CHUNK_FV(PI, PS)                                                        \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 0, true, true>(GdnArgs);   \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 0, false, true>(GdnArgs);  \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 2, true, true>(GdnArgs);   \
  GDN_KW_1 __global__ void k_chunk<GDN_C, GDN_D, PI, PS, 2, false, true>(GdnArgs);
GDN_EACH_PAIR(GDN_CHUNK_FV)
#endif
// part 2: the scans
#define GDN_SCAN_BWD(PI, PS, TIO) GDN_KW_2 __global__ void k_scan_bwd<GDN_C, GDN_D, kDVT, PI, PS, TIO>(GdnArgs);
#if GDN_C == 128 && GDN_D == 128
#define GDN_SCAN_FWD(PI, PS) GDN_KW_2 __global__ void k_scan_fwd_split<PI, PS>(GdnArgs);
#else
#define GDN_SCAN_FWD(PI, PS) GDN_KW_2 __global__ void k_scan_fwd<GDN_C, GDN_D, kDVT, PI, PS>(GdnArgs);
#endif
#define GDN_SCANS(PI, PS) \
  GDN_SCAN_FWD(PI, PS)    \
  GDN_EACH_IO(GDN_SCAN_BWD, PI, PS)
GDN_EACH_PAIR(GDN_SCANS)
// part 3: k_out, without and with the norm
#define GDN_OUT_IO(PI, PS, TIO)                                            \
  GDN_KW_3 __global__ void k_out<GDN_C, GDN_D, PI, PS, TIO, false>(GdnArgs); \
  GDN_KW_3 __global__ void k_out<GDN_C, GDN_D, PI, PS, TIO, true>(GdnArgs);
#define GDN_OUT(PI, PS) GDN_EACH_IO(GDN_OUT_IO, PI, PS)
GDN_EACH_PAIR(GDN_OUT)
#if GDN_C == 128 && GDN_D == 128  // and with q from the raw rows (bf16 I/O)
#define GDN_OUT_FQ(PI, PS)                                                                \
  GDN_KW_3 __global__ void k_out<GDN_C, GDN_D, PI, PS, uint16_t, false, true>(GdnArgs); \
  GDN_KW_3 __global__ void k_out<GDN_C, GDN_D, PI, PS, uint16_t, true, true>(GdnArgs);
GDN_EACH_PAIR(GDN_OUT_FQ)
#endif
// part 4: k_bwd_local (one A-side precision each: the pairs' first members, once)
#define GDN_LOCAL_IO(PI, PS, TIO) GDN_KW_4 __global__ void k_bwd_local<GDN_C, GDN_D, PI, TIO>(GdnArgs);
GDN_EACH_IO(GDN_LOCAL_IO, P_F32, 0)
GDN_EACH_IO(GDN_LOCAL_IO, P_BF16X3, 0)
GDN_EACH_IO(GDN_LOCAL_IO, P_BF16, 0)
// part 5: k_bwd_grads
#define GDN_GRADS_IO(PI, PS, TIO) GDN_KW_5 __global__ void k_bwd_grads<GDN_C, GDN_D, PI, PS, TIO>(GdnArgs);
#define GDN_GRADS(PI, PS) GDN_EACH_IO(GDN_GRADS_IO, PI, PS)
GDN_EACH_PAIR(GDN_GRADS)

#if GDN_PART == 0
namespace {

// compute units of the current device (queried once per device): the persistent kernels run
// one workgroup per CU
dim3 chunks_grid(const GdnArgs& A) { return dim3(A.B * A.H * A.N); }

int cu_count() {
  static int cache[16] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 16) dev = 0;
  if (!cache[dev]) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cache[dev] = c;
  }
  return cache[dev];
}

template <int C, int D, int PI, int PS, class TIO, class TG>
hipError_t run(const GdnArgs& A, hipStream_t st, int backward, const Timer* tm) {
  constexpr int DVT = D < 32 ? D : 32;
  constexpr int NS = (C > D ? C : D) * 4;
  const dim3 prep(A.B * A.N * (2 * A.Hk + A.H));  // the slot fastest (k_prep, k_post)
  const dim3 chunks(A.B * A.H * A.N);
  // the scans: (row, head, Dv tile) chains, each split into up to `parts` chunk ranges at
  // segment resets (rows without resets leave the extra ranges empty)
  const int chains = A.B * A.H * (D / DVT);
  int parts = (2 * cu_count() + chains - 1) / chains;
  parts = parts < 1 ? 1 : (parts > A.N ? A.N : parts);
  GdnArgs L = A;  // the launched arguments
  L.parts = parts;
  // bf16 I/O through a conv of 1 to 4 taps at C = D = 128: the forward's k_chunk builds the v
  // rows from the raw ones, and with one value head per key head k_out the q rows (with more,
  // it would build each q row once per value head: measured slower at 9B); k_prep skips them
  // (the backward's k_prep writes them)
  constexpr bool kFV = C == 128 && D == 128 && std::is_same_v<TIO, uint16_t>;
  L.fuse_v = A.fuse_v && kFV && !backward && A.taps >= 1 && A.taps <= 4;
  L.fuse_q = L.fuse_v && A.ratio == 1;
  // a workspace without fp32 q or v rows (gdn_api.hip's layout: the same rule) needs these
  // kernels to build them: fail rather than let k_prep write through a null pointer
  if (!backward && ((!L.fuse_v && !A.vv) || (!L.fuse_q && !A.qn))) return hipErrorInvalidValue;
  const dim3 tiles(chains * parts);
  const int units = A.B * A.H * A.N, cus = cu_count();
  const dim3 persist(units < cus ? units : cus);
  auto mark = [&](int k, int end) {
    if (tm) tm->mark(tm->self, k, end, st);
  };
#define GDN_LAUNCH(id, kern, grid, block)                  \
  do {                                                     \
    mark(id, 0);                                           \
    hipLaunchKernelGGL(kern, grid, block, 0, st, L);       \
    mark(id, 1);                                           \
  } while (0)
  if (!backward) {
    if (A.taps <= 4) GDN_LAUNCH(K_PREP_FWD, (k_prep<C, D, TIO, TG, 3>), prep, dim3(256));
    else GDN_LAUNCH(K_PREP_FWD, (k_prep<C, D, TIO, TG, 4>), prep, dim3(256));
    if (A.res == 0) {
      if (L.fuse_v) {
        if constexpr (kFV) {
          if (A.inv == 0) GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 0, true, true>), persist, dim3(C * 4));
          else GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 0, false, true>), persist, dim3(C * 4));
        }
      } else if (A.inv == 0) GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 0, true>), persist, dim3(C * 4));
      else GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 0, false>), persist, dim3(C * 4));
    } else {  // T kept for the backward
      if (L.fuse_v) {
        if constexpr (kFV) {
          if (A.inv == 0) GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 2, true, true>), persist, dim3(C * 4));
          else GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 2, false, true>), persist, dim3(C * 4));
        }
      } else if (A.inv == 0) GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 2, true>), persist, dim3(C * 4));
      else GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 2, false>), persist, dim3(C * 4));
    }
    if constexpr (C == 128 && D == 128) GDN_LAUNCH(K_SCAN_FWD, (k_scan_fwd_split<PI, PS>), tiles, dim3(512));
    else GDN_LAUNCH(K_SCAN_FWD, (k_scan_fwd<C, D, DVT, PI, PS>), tiles, dim3(NS));
    if (L.fuse_q) {
      if constexpr (kFV) {
        if (A.ny) GDN_LAUNCH(K_OUT, (k_out<C, D, PI, PS, TIO, true, true>), persist, dim3(C * 4));
        else GDN_LAUNCH(K_OUT, (k_out<C, D, PI, PS, TIO, false, true>), persist, dim3(C * 4));
      }
    } else if (A.ny) GDN_LAUNCH(K_OUT, (k_out<C, D, PI, PS, TIO, true>), persist, dim3(C * 4));
    else GDN_LAUNCH(K_OUT, (k_out<C, D, PI, PS, TIO>), persist, dim3(C * 4));
    if (A.final_state) GDN_LAUNCH(K_FINAL_STATE, (k_final_state<C, D>), dim3(A.B * A.H * (D / DVT)), dim3(256));
    if (A.conv_state && A.taps > 1) GDN_LAUNCH(K_FINAL_STATE, (k_conv_state<TIO>), dim3(A.B), dim3(256));
  } else {
    const int wouts = A.d_conv_w ? A.taps * A.W : 0;  // one workgroup per head, then the conv weights
    if (A.taps <= 4) GDN_LAUNCH(K_PREP_BWD, (k_prep<C, D, TIO, TG, 3>), prep, dim3(256));
    else GDN_LAUNCH(K_PREP_BWD, (k_prep<C, D, TIO, TG, 4>), prep, dim3(256));
    if (A.res == 0) {  // T and v_new rebuilt
      if (A.inv == 0) GDN_LAUNCH(K_CHUNK_BWD, (k_chunk<C, D, PI, PS, 1, true>), persist, dim3(C * 4));
      else GDN_LAUNCH(K_CHUNK_BWD, (k_chunk<C, D, PI, PS, 1, false>), persist, dim3(C * 4));
    } else if (A.res == 1) {  // v_new from the saved T
      GDN_LAUNCH(K_CHUNK_BWD, (k_chunk<C, D, PI, PS, 3, false>), persist, dim3(C * 4));
    }  // else both saved
    GDN_LAUNCH(K_BWD_LOCAL, (k_bwd_local<C, D, PI, TIO>), persist, dim3(C * 4));
    GDN_LAUNCH(K_SCAN_BWD, (k_scan_bwd<C, D, DVT, PI, PS, TIO>), tiles, dim3(NS));
    GDN_LAUNCH(K_BWD_GRADS, (k_bwd_grads<C, D, PI, PS, TIO>), chunks, dim3(C * 4));
    // the conv halo sized to the taps (taps - 1 <= 3 for the model's conv of 4); d(conv w)
    // accumulated only when it is wanted
    const bool dw = A.d_conv_w && A.taps > 0;
    if (A.taps <= 4) {
      if (dw) GDN_LAUNCH(K_POST, (k_post<C, D, TIO, TG, 3, true>), prep, dim3(256));
      else GDN_LAUNCH(K_POST, (k_post<C, D, TIO, TG, 3, false>), prep, dim3(256));
    } else {
      if (dw) GDN_LAUNCH(K_POST, (k_post<C, D, TIO, TG, 4, true>), prep, dim3(256));
      else GDN_LAUNCH(K_POST, (k_post<C, D, TIO, TG, 4, false>), prep, dim3(256));
    }
    GDN_LAUNCH(K_REDUCE, (k_reduce<C>), dim3(A.H + (wouts + 255) / 256), dim3(256));
  }
#undef GDN_LAUNCH
  return hipGetLastError();
}

// the v2 operator: its own ends (k_prep_v2, k_post_v2) around the same middle kernels
template <int C, int D, int PI, int PS, class TIO, class TQK, class TG>
hipError_t run_v2(const GdnArgs& A, hipStream_t st, int backward, const Timer* tm) {
  constexpr int DVT = D < 32 ? D : 32;
  constexpr int NS = (C > D ? C : D) * 4;
  const dim3 ends(A.B * A.N, 2 * A.Hk + A.H);
  const int chains = A.B * A.H * (D / DVT);
  int parts = (2 * cu_count() + chains - 1) / chains;
  parts = parts < 1 ? 1 : (parts > A.N ? A.N : parts);
  GdnArgs L = A;
  L.parts = parts;
  L.fuse_v = 0;  // v is an input here (k_prep_v2 writes its rows)
  L.fuse_q = 0;
  const dim3 tiles(chains * parts);
  const int units = A.B * A.H * A.N, cus = cu_count();
  const dim3 persist(units < cus ? units : cus);
  auto mark = [&](int k, int end) {
    if (tm) tm->mark(tm->self, k, end, st);
  };
#define GDN_LAUNCH(id, kern, grid, block)                  \
  do {                                                     \
    mark(id, 0);                                           \
    hipLaunchKernelGGL(kern, grid, block, 0, st, L);       \
    mark(id, 1);                                           \
  } while (0)
  if (!backward) {
    GDN_LAUNCH(K_PREP_FWD, (k_prep_v2<C, D, TIO, TQK, TG>), ends, dim3(256));
    if (A.res == 0) {
      if (A.inv == 0) GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 0, true>), persist, dim3(C * 4));
      else GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 0, false>), persist, dim3(C * 4));
    } else {
      if (A.inv == 0) GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 2, true>), persist, dim3(C * 4));
      else GDN_LAUNCH(K_CHUNK_FWD, (k_chunk<C, D, PI, PS, 2, false>), persist, dim3(C * 4));
    }
    if constexpr (C == 128 && D == 128) GDN_LAUNCH(K_SCAN_FWD, (k_scan_fwd_split<PI, PS>), tiles, dim3(512));
    else GDN_LAUNCH(K_SCAN_FWD, (k_scan_fwd<C, D, DVT, PI, PS>), tiles, dim3(NS));
    GDN_LAUNCH(K_OUT, (k_out<C, D, PI, PS, TIO>), persist, dim3(C * 4));
    if (A.final_state) GDN_LAUNCH(K_FINAL_STATE, (k_final_state<C, D>), dim3(A.B * A.H * (D / DVT)), dim3(256));
  } else {
    GDN_LAUNCH(K_PREP_BWD, (k_prep_v2<C, D, TIO, TQK, TG>), ends, dim3(256));
    if (A.res == 0) {
      if (A.inv == 0) GDN_LAUNCH(K_CHUNK_BWD, (k_chunk<C, D, PI, PS, 1, true>), persist, dim3(C * 4));
      else GDN_LAUNCH(K_CHUNK_BWD, (k_chunk<C, D, PI, PS, 1, false>), persist, dim3(C * 4));
    } else if (A.res == 1) {
      GDN_LAUNCH(K_CHUNK_BWD, (k_chunk<C, D, PI, PS, 3, false>), persist, dim3(C * 4));
    }
    GDN_LAUNCH(K_BWD_LOCAL, (k_bwd_local<C, D, PI, TIO>), persist, dim3(C * 4));
    GDN_LAUNCH(K_SCAN_BWD, (k_scan_bwd<C, D, DVT, PI, PS, TIO>), tiles, dim3(NS));
    GDN_LAUNCH(K_BWD_GRADS, (k_bwd_grads<C, D, PI, PS, TIO>), chunks_grid(A), dim3(C * 4));
    GDN_LAUNCH(K_POST, (k_post_v2<C, D, TIO, TQK, TG>), ends, dim3(256));
  }
#undef GDN_LAUNCH
  return hipGetLastError();
}

template <int PI, int PS>
void fill_v2(GdnFn (&f)[2][2][2]) {
  f[0][0][0] = run_v2<GDN_C, GDN_D, PI, PS, float, float, float>;
  f[0][0][1] = run_v2<GDN_C, GDN_D, PI, PS, float, float, uint16_t>;
  f[0][1][0] = run_v2<GDN_C, GDN_D, PI, PS, float, uint16_t, float>;
  f[0][1][1] = run_v2<GDN_C, GDN_D, PI, PS, float, uint16_t, uint16_t>;
  f[1][0][0] = run_v2<GDN_C, GDN_D, PI, PS, uint16_t, float, float>;
  f[1][0][1] = run_v2<GDN_C, GDN_D, PI, PS, uint16_t, float, uint16_t>;
  f[1][1][0] = run_v2<GDN_C, GDN_D, PI, PS, uint16_t, uint16_t, float>;
  f[1][1][1] = run_v2<GDN_C, GDN_D, PI, PS, uint16_t, uint16_t, uint16_t>;
}

template <int PI, int PS>
void fill(GdnFn (&f)[2][2]) {
  f[0][0] = run<GDN_C, GDN_D, PI, PS, float, float>;
  f[0][1] = run<GDN_C, GDN_D, PI, PS, float, uint16_t>;
  f[1][0] = run<GDN_C, GDN_D, PI, PS, uint16_t, float>;
  f[1][1] = run<GDN_C, GDN_D, PI, PS, uint16_t, uint16_t>;
}

ShapeTable make() {
  ShapeTable t{};
  t.C = GDN_C;
  t.D = GDN_D;
  fill<P_F32, P_F32>(t.fn[0]);       // highest
  fill<P_BF16X3, P_BF16X3>(t.fn[1]); // high
  fill<P_BF16, P_BF16>(t.fn[2]);     // bf16
  fill<P_BF16X3, P_BF16>(t.fn[3]);   // mixed
  fill_v2<P_F32, P_F32>(t.fnv2[0]);
  fill_v2<P_BF16X3, P_BF16X3>(t.fnv2[1]);
  fill_v2<P_BF16, P_BF16>(t.fnv2[2]);
  fill_v2<P_BF16X3, P_BF16>(t.fnv2[3]);
  return t;
}

}  // namespace

#define GDN_CAT_(a, b, c) a##b##_##c
#define GDN_CAT(a, b, c) GDN_CAT_(a, b, c)
const ShapeTable* GDN_CAT(table_, GDN_C, GDN_D)() {
  static const ShapeTable t = make();
  return &t;
}
#endif  // GDN_PART == 0

}  // namespace gdn
