// Device building blocks of the GDN megakernel for gfx950 (MI355X, CDNA4).
//
// Matrix products run on 16x16 MFMA tiles, one wave (64 lanes) per tile strip. A lane's
// operand fragment is 8 consecutive contraction values: A(i, k0 + 8*(lane/16) + e) and
// B(k0 + 8*(lane/16) + e, j) for e = 0..7, with i = i0 + lane%16 and j = j0 + lane%16.
// The accumulator of a tile holds D[4*(lane/16) + r][lane%16], r = 0..3.
//
// Three arithmetic modes (the reference's "precision", xla.py:23-36):
//   P_F32    fp32 operands on v_mfma_f32_16x16x4_f32 (8 instructions per 32 k-values)
//   P_BF16X3 each fp32 operand split into bf16 hi + lo, hi*hi + hi*lo + lo*hi on
//            v_mfma_f32_16x16x32_bf16, fp32 accumulation (the TPU's bf16_3x "high")
//   P_BF16   one bf16 pass with fp32 accumulation
// Operands are "views": small structs whose load(r, k, out) fills out[e] = V(r, k + e).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace gdn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum : int { P_F32 = 0, P_BF16X3 = 1, P_BF16 = 2, P_X3_BEXACT = 3, P_X3_AEXACT = 4 };
// P_X3_BEXACT / P_X3_AEXACT: a bf16x3 product whose B (A) operand holds bf16 values exactly (its
// low plane is zero, e.g. a bf16 activation): the pass that multiplies by that low plane only
// adds exact zeros and is skipped, so the result is the bf16x3 one. The other operand is split.
template <int P> constexpr int a_prec() { return P == P_X3_BEXACT ? P_BF16X3 : P == P_X3_AEXACT ? P_BF16 : P; }
template <int P> constexpr int b_prec() { return P == P_X3_BEXACT ? P_BF16 : P == P_X3_AEXACT ? P_BF16X3 : P; }
// the bf16x3 product when the operands are stored as x (its tiles' precision when bf16-exact)
template <int P, bool EXACT_B> constexpr int exact_b() { return P == P_BF16X3 && EXACT_B ? P_X3_BEXACT : P; }
template <int P, bool EXACT_A> constexpr int exact_a() { return P == P_BF16X3 && EXACT_A ? P_X3_AEXACT : P; }

__device__ __forceinline__ int lane() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave() { return threadIdx.x >> 6; }
// The 16-row strip of a wave in the kernels with one strip per wave (NW = C/16 waves), as a
// wave-uniform value. A workgroup's waves w and w + 4 run on one SIMD (gfx950 gives the first
// four waves one SIMD each, in an order that rotates between workgroups, and the next four the
// same SIMDs in the same order), and strip s carries s + 1 tiles of a product over the
// triangle's rows (NW - s of one over its columns). PAIR puts strips s and NW - 1 - s on one
// SIMD, which then carries NW + 1 tiles of every such product (without it: 6, 8, 10 and 12 for
// NW = 8). readfirstlane marks the value uniform: the strip-dependent loop bounds and branches
// are otherwise compiled as divergent code.
// A wave-uniform value made opaque to the optimiser at this point (it stays in a scalar
// register). Inside a persistent kernel's unit loop, the strip index taken through it keeps the
// conditions on it (tile t below, on or above the strip's diagonal ...) from being computed
// once before the loop and held across it as 64-bit lane masks, which run the kernel out of
// scalar registers and spill them to vector lanes.
__device__ __forceinline__ int opaque_uniform(int v) {
  asm volatile("" : "+s"(v));
  return v;
}
template <int NW, bool PAIR>
__device__ __forceinline__ int wave_strip() {
  const int w = wave();
  return __builtin_amdgcn_readfirstlane(PAIR && NW == 8 && w >= 4 ? 11 - w : w);
}

// ---------------------------------------------------------------- debug: poisoned LDS
// Built with -DGDN_LDS_POISON (the debug library libtjev_gdn_lds_poison.so), every kernel first
// fills each LDS array it declares with all-ones bytes (NaN as fp32 and as bf16, -1 as an int)
// and synchronises, so a read of LDS that the kernel did not write carries NaN into its results
// (the reference's interpret-mode run with uninitialized_memory="nan", pallas_tpu.py:209-219).
// Without the flag the macro is empty.
#ifdef GDN_LDS_POISON
__device__ __forceinline__ void poison_bytes(void* p, unsigned n) {
  uint32_t* w = static_cast<uint32_t*>(p);
  for (unsigned i = threadIdx.x; i < n / 4; i += blockDim.x) w[i] = 0xffffffffu;
  unsigned char* c = static_cast<unsigned char*>(p);
  for (unsigned i = n / 4 * 4 + threadIdx.x; i < n; i += blockDim.x) c[i] = 0xff;
}
template <class... Ts>
__device__ __forceinline__ void poison_lds(Ts&... xs) {
  (poison_bytes(static_cast<void*>(&xs), (unsigned)sizeof(xs)), ...);
  __syncthreads();
}
#define GDN_POISON_LDS(...) ::gdn::poison_lds(__VA_ARGS__)
#else
#define GDN_POISON_LDS(...) ((void)0)
#endif

// ---------------------------------------------------------------- bf16 storage
// bf16 tensors are held as uint16_t; conversion rounds to nearest even (as torch does).
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }
// (gfx950's v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN)
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// A single fp32 store into LDS that the backend may not pair with its neighbours. ROCm 7.2's
// SI load/store optimizer can merge two such stores into one ds_write2_b32 with a wrongly
// scaled first offset (seen for 272/336-byte offsets: emitted as 17/84 dwords); the empty asm
// with a memory clobber keeps every store single. build.py checks the merged DS accesses of
// every kernel for this.
__device__ __forceinline__ void lds_st(float* p, float v) {
  *p = v;
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ float ldf(const float* p) { return *p; }
__device__ __forceinline__ float ldf(const uint16_t* p) { return bf2f(*p); }
__device__ __forceinline__ void stf(float* p, float v) { *p = v; }
__device__ __forceinline__ void stf(uint16_t* p, float v) { *p = f2bf(v); }

// 4 consecutive elements (8-byte aligned for bf16, 16-byte for fp32)
__device__ __forceinline__ void st4_io(float* p, const float (&v)[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void st4_io(uint16_t* p, const float (&v)[4]) {
  *reinterpret_cast<uint2*>(p) = make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16),
                                            (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16));
}

// 8 consecutive elements (16-byte aligned for bf16, 32-byte for fp32) as floats
__device__ __forceinline__ void ld8(const float* p, float (&o)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
}
__device__ __forceinline__ void ld8(const uint16_t* p, float (&o)[8]) {
  const uint4 a = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[2 * e] = __uint_as_float(w[e] << 16);
    o[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
}

// 8 consecutive values stored as T (bf16 rounds to nearest even)
__device__ __forceinline__ void st8_io(float* p, const float (&v)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void st8_io(uint16_t* p, const float (&v)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = (uint32_t)f2bf(v[2 * e]) | ((uint32_t)f2bf(v[2 * e + 1]) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
// Nontemporal forms for the step's final outputs, which no later kernel of the step reads:
// they are not kept in the caches the next kernels' inputs go through
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void st8_io_nt(float* p, const float (&v)[8]) {
  const f32x4 a = {v[0], v[1], v[2], v[3]}, b = {v[4], v[5], v[6], v[7]};
  __builtin_nontemporal_store(a, reinterpret_cast<f32x4*>(p));
  __builtin_nontemporal_store(b, reinterpret_cast<f32x4*>(p) + 1);
}
__device__ __forceinline__ void st8_io_nt(uint16_t* p, const float (&v)[8]) {
  u32x4 w;
  w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
  w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
  w.z = (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16);
  w.w = (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16);
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
}

// 8 consecutive stored values held as loaded (bf16 stays packed), converted when used
template <class T> struct Raw8;
template <> struct Raw8<float> {
  float4 a, b;
  __device__ __forceinline__ void load(const float* p) {
    a = reinterpret_cast<const float4*>(p)[0];
    b = reinterpret_cast<const float4*>(p)[1];
  }
  __device__ __forceinline__ void get(float (&o)[8]) const {
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
};
template <> struct Raw8<uint16_t> {
  uint4 a;
  __device__ __forceinline__ void load(const uint16_t* p) { a = *reinterpret_cast<const uint4*>(p); }
  __device__ __forceinline__ void get(float (&o)[8]) const {
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[2 * e] = __uint_as_float(w[e] << 16);
      o[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
    }
  }
};

// 4 consecutive stored values held as loaded (8-byte aligned for bf16, 16-byte for fp32)
template <class T> struct Raw4;
template <> struct Raw4<float> {
  float4 a;
  __device__ __forceinline__ void load(const float* p) { a = *reinterpret_cast<const float4*>(p); }
  __device__ __forceinline__ void get(float (&o)[4]) const { o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; }
};
template <> struct Raw4<uint16_t> {
  uint2 a;
  __device__ __forceinline__ void load(const uint16_t* p) { a = *reinterpret_cast<const uint2*>(p); }
  __device__ __forceinline__ float elem(int e) const {  // value e (a compile-time index)
    const uint32_t w = e < 2 ? a.x : a.y;
    return __uint_as_float(e % 2 ? w & 0xffff0000u : w << 16);
  }
  __device__ __forceinline__ void get(float (&o)[4]) const {
    o[0] = __uint_as_float(a.x << 16);
    o[1] = __uint_as_float(a.x & 0xffff0000u);
    o[2] = __uint_as_float(a.y << 16);
    o[3] = __uint_as_float(a.y & 0xffff0000u);
  }
};
// 4 consecutive stored values as loaded: a float4, or 4 bf16 packed in a uint2 (expanded exactly
// when used, so the load's latency is not waited for at the load)
template <class T>
using Packed4 = std::conditional_t<sizeof(T) == 2, uint2, float4>;
__device__ __forceinline__ float4 f4_of(const float4& v) { return v; }
__device__ __forceinline__ float4 f4_of(const uint2& v) {
  return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                     __uint_as_float(v.y & 0xffff0000u));
}
// a value rounded to the storage type T and back (bf16: round to nearest even)
template <class T>
__device__ __forceinline__ float rnd_io(float v) {
  if constexpr (sizeof(T) == 2) {
    return bf2f(f2bf(v));
  } else {
    return v;
  }
}

// ---------------------------------------------------------------- numerics
__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
// The elementwise activations' forms on the hardware transcendentals (v_exp_f32, v_rcp_f32,
// v_rsq_f32: about 1 ulp each, a few ulp composed), used on bf16 activations.
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }
__device__ __forceinline__ float sigmoid_fast(float x) { return __builtin_amdgcn_rcpf(1.0f + exp_fast(-x)); }
__device__ __forceinline__ float rsqrt_fast(float x) { return __builtin_amdgcn_rsqf(x); }
// the sigmoid of an activation stored as T: the hardware form for bf16 activations (whose own
// rounding is 2^-9), the correctly rounded one for fp32 (the fp32 parity path)
template <class T>
__device__ __forceinline__ float sigmoid_io(float x) {
  if constexpr (sizeof(T) == 2) {
    return sigmoid_fast(x);
  } else {
    return sigmoidf_(x);
  }
}
template <class T>
__device__ __forceinline__ float rsqrt_io(float x) {
  if constexpr (sizeof(T) == 2) {
    return rsqrt_fast(x);
  } else {
    return 1.0f / sqrtf(x);
  }
}
// jax.nn.softplus = logaddexp(x, 0) = max(x, 0) + log1p(exp(-|x|))
__device__ __forceinline__ float softplusf_(float x) {
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}

// ---------------------------------------------------------------- MFMA fragments
template <int P> struct Frag;
template <> struct Frag<P_F32> { float v[8]; };
template <> struct Frag<P_BF16> { bf16x8 hi; };
template <> struct Frag<P_BF16X3> { bf16x8 hi, lo; };

template <int P>
__device__ __forceinline__ Frag<P> make_frag(const float (&x)[8]) {
  Frag<P> f;
  if constexpr (P == P_F32) {
#pragma unroll
    for (int e = 0; e < 8; ++e) f.v[e] = x[e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) f.hi[e] = (__bf16)x[e];
    if constexpr (P == P_BF16X3) {
#pragma unroll
      for (int e = 0; e < 8; ++e) f.lo[e] = (__bf16)(x[e] - (float)f.hi[e]);
    }
  }
  return f;
}

template <int P>
__device__ __forceinline__ void mma(f32x4& acc, const Frag<a_prec<P>()>& a, const Frag<b_prec<P>()>& b) {
  if constexpr (P == P_F32) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[e], b.v[e], acc, 0, 0, 0);
  } else if constexpr (P == P_BF16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, acc, 0, 0, 0);
  } else if constexpr (P == P_X3_BEXACT) {  // as bf16x3 without the a.hi * b.lo = 0 pass
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, acc, 0, 0, 0);
  } else if constexpr (P == P_X3_AEXACT) {  // as bf16x3 without the a.lo * b.hi = 0 pass
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, acc, 0, 0, 0);
  } else {  // the small cross terms first, then hi*hi
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, acc, 0, 0, 0);
  }
}

// ---------------------------------------------------------------- operand views
// V(r, k) = p[r*ld + k]: the contraction index is contiguous (vector loads).
template <class T>
struct KRow {
  const T* p;
  int ld;
  __device__ __forceinline__ void load(int r, int k, float (&o)[8]) const { ld8(p + r * ld + k, o); }
};
// V(r, k) = p[k*ld + r]: the contraction index is the row (strided loads; LDS operands).
template <class T>
struct KCol {
  const T* p;
  int ld;
  __device__ __forceinline__ void load(int r, int k, float (&o)[8]) const {
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = ldf(p + (k + e) * ld + r);
  }
};
// V'(r, k) = c * s[r] * V(r, k)
template <class V>
struct ScaleR {
  V v;
  const float* s;
  float c;
  __device__ __forceinline__ void load(int r, int k, float (&o)[8]) const {
    v.load(r, k, o);
    const float f = c * s[r];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= f;
  }
};
// V'(r, k) = c * s[k] * V(r, k)
template <class V>
struct ScaleK {
  V v;
  const float* s;
  float c;
  __device__ __forceinline__ void load(int r, int k, float (&o)[8]) const {
    v.load(r, k, o);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] *= c * s[k + e];
  }
};
// Every view also yields a converted fragment: frag<Q>(r, k) = make_frag<Q>(load(r, k)).
#define GDN_VIEW_FRAG                                                            \
  template <int Q>                                                               \
  __device__ __forceinline__ Frag<Q> frag(int r, int k) const {                  \
    float x_[8];                                                                 \
    this->load(r, k, x_);                                                        \
    return make_frag<Q>(x_);                                                     \
  }
template <class T> struct KRowF : KRow<T> { GDN_VIEW_FRAG };
template <class T> struct KColF : KCol<T> { GDN_VIEW_FRAG };
template <class V> struct ScaleRF : ScaleR<V> { GDN_VIEW_FRAG };
template <class V> struct ScaleKF : ScaleK<V> { GDN_VIEW_FRAG };

template <class T> __device__ __forceinline__ KRowF<T> krow(const T* p, int ld) { return {{p, ld}}; }
template <class T> __device__ __forceinline__ KColF<T> kcol(const T* p, int ld) { return {{p, ld}}; }
template <class V> __device__ __forceinline__ ScaleRF<V> scale_r(V v, const float* s, float c = 1.f) { return {{v, s, c}}; }
template <class V> __device__ __forceinline__ ScaleKF<V> scale_k(V v, const float* s, float c = 1.f) { return {{v, s, c}}; }


// ---------------------------------------------------------------- pre-converted LDS operands
// two values as bf16 (round to nearest even) in one 32-bit word, the first in the low half
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) | ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}
// v - bf16(v): the part a bf16 pass drops (exact in fp32)
__device__ __forceinline__ float lo_part(float v) { return v - (float)(__bf16)v; }

// Op<P>: an operand tile in LDS, converted once when it is staged. Element (r, k) sits at
// r*ld + k with the contraction index k contiguous (r: the M index of an A operand, the N index
// of a B operand), so a fragment is one 16-byte read per plane. P_F32 keeps fp32; P_BF16 one bf16
// plane; P_BF16X3 the bf16 hi and lo planes of each value. A P_BF16X3 tile also serves one-pass
// products (its hi plane), as the state-path products of "mixed" need.
template <int P> struct Op;
template <>
struct Op<P_F32> {
  float* p;
  int ld;
  __device__ __forceinline__ void put(int r, int k, float v) const { lds_st(p + r * ld + k, v); }
  // two consecutive k (k even), four consecutive k (k a multiple of 4)
  __device__ __forceinline__ void put2(int r, int k, float v0, float v1) const {
    *reinterpret_cast<float2*>(p + r * ld + k) = make_float2(v0, v1);
    asm volatile("" ::: "memory");
  }
  __device__ __forceinline__ void put4(int r, int k, float v0, float v1, float v2, float v3) const {
    *reinterpret_cast<float4*>(p + r * ld + k) = make_float4(v0, v1, v2, v3);
  }
  // eight consecutive k (k a multiple of 8)
  __device__ __forceinline__ void put8(int r, int k, const float (&v)[8]) const {
    *reinterpret_cast<float4*>(p + r * ld + k) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + r * ld + k + 4) = make_float4(v[4], v[5], v[6], v[7]);
  }
  template <int Q>
  __device__ __forceinline__ Frag<Q> frag(int r, int k) const {
    static_assert(Q == P_F32, "an fp32 tile feeds fp32 products");
    float x[8];
    ld8(p + r * ld + k, x);
    Frag<P_F32> f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f.v[e] = x[e];
    return f;
  }
};
template <>
struct Op<P_BF16> {
  uint16_t* hi;
  int ld;
  __device__ __forceinline__ void put(int r, int k, float v) const {
    hi[r * ld + k] = __builtin_bit_cast(uint16_t, (__bf16)v);
  }
  __device__ __forceinline__ void put2(int r, int k, float v0, float v1) const {
    *reinterpret_cast<uint32_t*>(hi + r * ld + k) = pack2(v0, v1);
  }
  __device__ __forceinline__ void put4(int r, int k, float v0, float v1, float v2, float v3) const {
    *reinterpret_cast<uint2*>(hi + r * ld + k) = make_uint2(pack2(v0, v1), pack2(v2, v3));
  }
  __device__ __forceinline__ void put8(int r, int k, const float (&v)[8]) const {
    *reinterpret_cast<uint4*>(hi + r * ld + k) =
        make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
  }
  template <int Q>
  __device__ __forceinline__ Frag<Q> frag(int r, int k) const {
    static_assert(Q == P_BF16, "a bf16 tile feeds one-pass products");
    Frag<P_BF16> f;
    f.hi = *reinterpret_cast<const bf16x8*>(hi + r * ld + k);
    return f;
  }
};
template <>
struct Op<P_BF16X3> {
  uint16_t* hi;
  uint16_t* lo;
  int ld;
  __device__ __forceinline__ void put(int r, int k, float v) const {
    const __bf16 h = (__bf16)v;
    hi[r * ld + k] = __builtin_bit_cast(uint16_t, h);
    lo[r * ld + k] = __builtin_bit_cast(uint16_t, (__bf16)(v - (float)h));
  }
  __device__ __forceinline__ void put2(int r, int k, float v0, float v1) const {
    *reinterpret_cast<uint32_t*>(hi + r * ld + k) = pack2(v0, v1);
    *reinterpret_cast<uint32_t*>(lo + r * ld + k) = pack2(lo_part(v0), lo_part(v1));
  }
  // bf16-exact values: the high plane only (the tile then feeds P_X3_BEXACT products)
  __device__ __forceinline__ void put2_hi(int r, int k, float v0, float v1) const {
    *reinterpret_cast<uint32_t*>(hi + r * ld + k) = pack2(v0, v1);
  }
  __device__ __forceinline__ void put4(int r, int k, float v0, float v1, float v2, float v3) const {
    *reinterpret_cast<uint2*>(hi + r * ld + k) = make_uint2(pack2(v0, v1), pack2(v2, v3));
    *reinterpret_cast<uint2*>(lo + r * ld + k) =
        make_uint2(pack2(lo_part(v0), lo_part(v1)), pack2(lo_part(v2), lo_part(v3)));
  }
  __device__ __forceinline__ void put8(int r, int k, const float (&v)[8]) const {
    *reinterpret_cast<uint4*>(hi + r * ld + k) =
        make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
    *reinterpret_cast<uint4*>(lo + r * ld + k) =
        make_uint4(pack2(lo_part(v[0]), lo_part(v[1])), pack2(lo_part(v[2]), lo_part(v[3])),
                   pack2(lo_part(v[4]), lo_part(v[5])), pack2(lo_part(v[6]), lo_part(v[7])));
  }
  template <int Q>
  __device__ __forceinline__ Frag<Q> frag(int r, int k) const {
    static_assert(Q == P_BF16X3 || Q == P_BF16, "a split tile feeds bf16x3 or one-pass products");
    Frag<Q> f;
    f.hi = *reinterpret_cast<const bf16x8*>(hi + r * ld + k);
    if constexpr (Q == P_BF16X3) f.lo = *reinterpret_cast<const bf16x8*>(lo + r * ld + k);
    return f;
  }
};

// LDS bytes and carving of an R x K operand tile (16 bytes of padding per row)
template <int P, int R, int K>
struct OpTile {
  static constexpr int LD = K + 8;
  static constexpr int BYTES = R * LD * (P == P_BF16 ? 2 : 4);
  __device__ __forceinline__ static Op<P> at(char* base) {
    if constexpr (P == P_F32) {
      return Op<P_F32>{reinterpret_cast<float*>(base), LD};
    } else if constexpr (P == P_BF16) {
      return Op<P_BF16>{reinterpret_cast<uint16_t*>(base), LD};
    } else {
      return Op<P_BF16X3>{reinterpret_cast<uint16_t*>(base), reinterpret_cast<uint16_t*>(base + R * LD * 2), LD};
    }
  }
};

template <int P>
__device__ __forceinline__ Frag<P> zero_frag() {
  float x[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  return make_frag<P>(x);
}

// ---------------------------------------------------------------- strip product
// acc[t] += fa . B(j0 + 16t + lane%16, kk) for the tiles t < tn: tiles in groups of up to four
// whose B fragments are all read before their products, one branch per group. tn is
// wave-uniform; the tiles of a partly used group (t >= tn) are computed too, and callers
// passing tn < TN ignore them.
template <int P, int TN, class BV>
__device__ __forceinline__ void tile_row(f32x4 (&acc)[TN], const Frag<a_prec<P>()>& fa, const BV& B, int j0, int kk,
                                         bool ok, int tn) {
  constexpr int G = TN < 4 ? TN : 4;
  constexpr int PB = b_prec<P>();
  static_assert(TN % G == 0, "tiles in whole groups");
  const int r = lane() & 15;
#pragma unroll
  for (int g = 0; g < TN / G; ++g) {
    if (G * g < tn) {
      Frag<PB> fb[G];
#pragma unroll
      for (int e = 0; e < G; ++e) fb[e] = ok ? B.template frag<PB>(j0 + 16 * (G * g + e) + r, kk) : zero_frag<PB>();
#pragma unroll
      for (int e = 0; e < G; ++e) mma<P>(acc[G * g + e], fa, fb[e]);
    }
  }
}

// acc[t] += sum over k in [kb, ke) of A(i0 + lane%16, k) * B(k, j0 + 16t + lane%16) for the
// tiles t < tn (see tile_row). kb is a multiple of 32; ke <= K. K is a multiple of 16; when K
// is 16 the lanes of the upper contraction half feed zeros. A and B are views (converted on
// use) or Op tiles (pre-converted).
template <int P, int K, int TN, class AV, class BV>
__device__ __forceinline__ void strip_mma(f32x4 (&acc)[TN], const AV& A, int i0, const BV& B, int j0,
                                          int kb = 0, int ke = K, int tn = TN) {
  const int l = lane();
  const int r = l & 15;
  const int kg = (l >> 4) << 3;
  for (int k = kb; k < ke; k += 32) {
    const bool ok = (K % 32 == 0) || (k + kg < K);
    constexpr int PA = a_prec<P>();
    const Frag<PA> fa = ok ? A.template frag<PA>(i0 + r, k + kg) : zero_frag<PA>();
    tile_row<P, TN>(acc, fa, B, j0, k + kg, ok, tn);
  }
}

// acc[t] += sum over k < K of A(i0 + 16t + lane%16, k) * B(k, j0 + lane%16) for TM 16-row tiles
// t of one 16-column tile: each B fragment is read once for the TM products.
template <int P, int K, int TM, class AV, class BV>
__device__ __forceinline__ void col_mma(f32x4 (&acc)[TM], const AV& A, int i0, const BV& B, int j0) {
  constexpr int PA = a_prec<P>(), PB = b_prec<P>();
  const int l = lane();
  const int r = l & 15;
  const int kg = (l >> 4) << 3;
#pragma unroll
  for (int k = 0; k < K; k += 32) {
    const bool ok = (K % 32 == 0) || (k + kg < K);
    const Frag<PB> fb = ok ? B.template frag<PB>(j0 + r, k + kg) : zero_frag<PB>();
    Frag<PA> fa[TM];
#pragma unroll
    for (int t = 0; t < TM; ++t) fa[t] = ok ? A.template frag<PA>(i0 + 16 * t + r, k + kg) : zero_frag<PA>();
#pragma unroll
    for (int t = 0; t < TM; ++t) mma<P>(acc[t], fa[t], fb);
  }
}

template <int TN>
__device__ __forceinline__ void zero(f32x4 (&acc)[TN]) {
#pragma unroll
  for (int t = 0; t < TN; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
}

// Row (within a 16-row strip) of accumulator element rr, and column within a tile.
__device__ __forceinline__ int acc_row(int rr) { return ((lane() >> 4) << 2) + rr; }
__device__ __forceinline__ int acc_col() { return lane() & 15; }

// contraction range of a lower-triangular left operand for rows [i0, i0+16): k <= i0+15
template <int K> __device__ __forceinline__ int tri_end(int i0) { return min(K, ((i0 + 16 + 31) / 32) * 32); }
// ... and of an upper-triangular one (a transposed lower-triangular): k >= i0
__device__ __forceinline__ int tri_begin(int i0) { return (i0 / 32) * 32; }

// v of another lane of the same 16-lane row by a DPP control (quad permutes, mirrors)
template <int CTRL>
__device__ __forceinline__ float dpp_read(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// 4 x 4 transpose within each quad of lanes: lane q of the quad holds v[r] = M[r][q] before
// and v[c] = M[q][c] after, by two exchanges of 2 x 2 blocks (quad permutes). Applied to an
// accumulator tile, lane (g, 4m + q) then holds row 4g + q, columns 4m .. 4m + 3.
__device__ __forceinline__ void quad_transpose(float (&v)[4]) {
  const int q = lane() & 3;
  const bool odd = q & 1, hi = q & 2;
  const float r0 = dpp_read<0xB1>(odd ? v[0] : v[1]), r2 = dpp_read<0xB1>(odd ? v[2] : v[3]);  // lane q ^ 1
  const float n0 = odd ? r0 : v[0], n1 = odd ? v[1] : r0, n2 = odd ? r2 : v[2], n3 = odd ? v[3] : r2;
  const float u0 = dpp_read<0x4E>(hi ? n0 : n2), u1 = dpp_read<0x4E>(hi ? n1 : n3);  // lane q ^ 2
  v[0] = hi ? u0 : n0;
  v[1] = hi ? u1 : n1;
  v[2] = hi ? n2 : u0;
  v[3] = hi ? n3 : u1;
}

// A 16 x 16 fp32 accumulator tile stored row-major at p (its element (0, 0); row stride ld) as
// it lies: 4 rows of one column per lane, 64-byte row segments per store. (A quad transpose
// first would make them 16-byte stores of 4 columns, at 14 VALU instructions per tile: slower
// wherever the storing wave's VALU work is on the kernel's critical path, as in the scans.)
__device__ __forceinline__ void st_tile(float* p, int ld, const f32x4& a) {
#pragma unroll
  for (int rr = 0; rr < 4; ++rr) p[(unsigned)(acc_row(rr) * ld + acc_col())] = a[rr];
}

// sum over each aligned group of N consecutive lanes (N a power of two <= 64), in every lane
// of the group: within a 16-lane row by DPP (lane ^ 1, lane ^ 2 as quad permutes, then the
// row's half mirror and mirror, which pair the quads and the halves), across rows by xor
// shuffles
template <int N>
__device__ __forceinline__ float sum_lanes(float v) {
  if constexpr (N >= 2) v += dpp_read<0xB1>(v);   // quad_perm [1,0,3,2]
  if constexpr (N >= 4) v += dpp_read<0x4E>(v);   // quad_perm [2,3,0,1]
  if constexpr (N >= 8) v += dpp_read<0x141>(v);  // row_half_mirror
  if constexpr (N >= 16) v += dpp_read<0x140>(v); // row_mirror
  if constexpr (N >= 32) v += __shfl_xor(v, 16);
  if constexpr (N >= 64) v += __shfl_xor(v, 32);
  return v;
}
// sum over the 16 lanes that share lane/16 (one accumulator row across a tile's columns)
__device__ __forceinline__ float sum16(float v) { return sum_lanes<16>(v); }
__device__ __forceinline__ float sum64(float v) { return sum_lanes<64>(v); }

__device__ __forceinline__ double sum64d(double v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m);
  return v;
}

// ---------------------------------------------------------------- launch mapping
// Workgroups go to the 8 XCDs round-robin (id % 8). This remap gives each XCD a contiguous
// range of logical ids, so work items that share inputs (the Dv tiles of one head) land on
// the same XCD and its L2. Identity when the grid is not a multiple of 8.
__device__ __forceinline__ int xcd_remap(int bid, int grid) {
  if (grid % 8) return bid;
  return (bid % 8) * (grid / 8) + bid / 8;
}

}  // namespace gdn
