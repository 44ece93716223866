// Host-side driver of the C ABI's argument checks for the AddressSanitizer build
// (tests/test_asan_host.py): every entry point with bad, null, misaligned, unsupported and
// edge-case arguments, and the size queries over many shapes. Nothing reaches a kernel launch
// (every call fails validation or is given no workspace), so no GPU is touched. Exit status:
// the number of calls whose status differed from the expected one.
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/tjev_gdn.h"

static int g_bad = 0;

static void expect(int got, int want, const char* what) {
  const char* msg = tjev_gdn_last_error();
  if (got != want) {
    std::printf("MISMATCH %s: status %d, expected %d (%s)\n", what, got, want, msg ? msg : "(null)");
    ++g_bad;
  } else if (got && (!msg || !std::strlen(msg))) {
    std::printf("MISMATCH %s: status %d without a message\n", what, got);
    ++g_bad;
  }
}

static tjev_gdn_params params(int B, int T, int Hk, int D, int H, int taps, int C) {
  tjev_gdn_params p;
  std::memset(&p, 0, sizeof(p));
  p.batch = B;
  p.length = T;
  p.key_heads = Hk;
  p.key_dim = D;
  p.value_heads = H;
  p.value_dim = D;
  p.taps = taps;
  p.chunk = C;
  p.precision = TJEV_GDN_HIGH;
  return p;
}

// made-up 4 KiB-aligned addresses: never dereferenced by the checks
static void* fake(int i) { return reinterpret_cast<void*>(static_cast<uintptr_t>(4096) * (i + 1)); }
static void* odd(int i) { return reinterpret_cast<void*>(static_cast<uintptr_t>(4096) * (i + 1) + 8); }

int main() {
  tjev_gdn_params p = params(2, 300, 2, 16, 4, 4, 16);
  const void* f[32];
  for (int i = 0; i < 32; ++i) f[i] = fake(i);
  void* ws = fake(40);

  // parameters
  expect(tjev_gdn_check(nullptr), TJEV_GDN_EINVAL, "null params");
  expect(tjev_gdn_check(&p), 0, "valid params");
  {
    tjev_gdn_params q = p;
    q.precision = 9;
    expect(tjev_gdn_check(&q), TJEV_GDN_EINVAL, "precision");
    q = p;
    q.chunk = 24;
    expect(tjev_gdn_check(&q), TJEV_GDN_EINVAL, "chunk");
    q = p;
    q.value_heads = 3;
    expect(tjev_gdn_check(&q), TJEV_GDN_EINVAL, "head groups");
    q = p;
    q.key_dim = q.value_dim = 48;
    expect(tjev_gdn_check(&q), TJEV_GDN_EUNSUPPORTED, "head dim");
    q = p;
    q.value_dim = 32;
    expect(tjev_gdn_check(&q), TJEV_GDN_EUNSUPPORTED, "Dk != Dv");
    q = p;
    q.batch = 0;
    expect(tjev_gdn_check(&q), TJEV_GDN_EINVAL, "zero batch");
    q = p;
    q.length = 1 << 30;
    q.batch = 1 << 20;
    expect(tjev_gdn_check(&q), TJEV_GDN_EINVAL, "too large");
    expect((int)tjev_gdn_workspace_bytes(&q, 1), 0, "no size for a bad problem");
  }
  // size queries over the compiled shapes and ragged lengths
  const int shapes[][2] = {
#define GDN_SHAPE(c, d) {c, d},
#include "../../tjev_amd/csrc/gdn_shapes.def"
#undef GDN_SHAPE
  };
  for (auto& s : shapes)
    for (int T : {1, 7, 16, 100, 1023, 4096})
      for (int res = 0; res < 3; ++res) {
        tjev_gdn_params q = params(3, T, 2, s[1], 6, 4, s[0]);
        q.residuals = res;
        const size_t f0 = tjev_gdn_workspace_bytes(&q, 0), b0 = tjev_gdn_workspace_bytes(&q, 1);
        const size_t r0 = tjev_gdn_residual_bytes(&q), st = tjev_gdn_states_bytes(&q);
        if (!f0 || !b0 || !r0 || !st || st > r0) {
          std::printf("MISMATCH sizes C=%d D=%d T=%d res=%d: %zu %zu %zu %zu\n", s[0], s[1], T, res, f0, b0, r0, st);
          ++g_bad;
        }
      }

  // the megakernel
  expect(tjev_gdn_mega2_fwd(&p, nullptr, nullptr, f[1], f[2], (const float*)f[3], (const float*)f[4],
                            (const float*)f[5], (const int32_t*)f[6], fake(7), (float*)fake(8), ws, 0),
         TJEV_GDN_EINVAL, "fwd null qkv");
  expect(tjev_gdn_mega2_fwd(&p, nullptr, odd(0), f[1], f[2], (const float*)f[3], (const float*)f[4],
                            (const float*)f[5], (const int32_t*)f[6], fake(7), (float*)fake(8), ws, 0),
         TJEV_GDN_EINVAL, "fwd misaligned qkv");
  expect(tjev_gdn_mega2_fwd(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                            (const float*)f[5], (const int32_t*)f[6], fake(7), (float*)fake(8), ws, 0),
         TJEV_GDN_EWORKSPACE, "fwd no workspace");
  expect(tjev_gdn_mega2_bwd(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                            (const float*)f[5], (const int32_t*)f[6], (const float*)f[8], f[9], fake(10), fake(11),
                            fake(12), (float*)fake(13), (float*)fake(14), (float*)fake(15), ws, 0),
         TJEV_GDN_EWORKSPACE, "bwd no workspace");
  expect(tjev_gdn_mega2_bwd(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                            (const float*)f[5], (const int32_t*)f[6], (const float*)f[8], f[9], nullptr, fake(11),
                            fake(12), (float*)fake(13), (float*)fake(14), (float*)fake(15), ws, 0),
         TJEV_GDN_EINVAL, "bwd null d_qkv");
  {
    tjev_gdn_params m1 = params(2, 300, 2, 16, 4, 0, 16);
    expect(tjev_gdn_mega2_bwd(&m1, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4], nullptr,
                              (const int32_t*)f[6], (const float*)f[8], f[9], fake(10), fake(11), fake(12),
                              (float*)fake(13), (float*)fake(14), (float*)fake(15), ws, 0),
           TJEV_GDN_EINVAL, "mega1 conv weight gradient");
  }
  // continued sequences
  expect(tjev_gdn_mega2_fwd_cont(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                 (const float*)f[5], (const int32_t*)f[6], (const float*)fake(20), fake(21), fake(7),
                                 (float*)fake(8), (float*)fake(22), fake(23), ws, 0),
         TJEV_GDN_EWORKSPACE, "fwd_cont all states");
  expect(tjev_gdn_mega2_fwd_cont(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                 (const float*)f[5], (const int32_t*)f[6], (const float*)odd(20), nullptr, fake(7),
                                 (float*)fake(8), nullptr, nullptr, ws, 0),
         TJEV_GDN_EINVAL, "fwd_cont misaligned state");
  expect(tjev_gdn_mega2_fwd_normed(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                   (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, fake(24),
                                   (const float*)fake(25), 1e-6f, fake(7), fake(26), (float*)fake(8), nullptr, nullptr,
                                   ws, 0),
         TJEV_GDN_EWORKSPACE, "fwd_normed");
  expect(tjev_gdn_mega2_fwd_normed(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                   (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, odd(24),
                                   (const float*)fake(25), 1e-6f, fake(7), fake(26), (float*)fake(8), nullptr, nullptr,
                                   ws, 0),
         TJEV_GDN_EINVAL, "fwd_normed misaligned gate");
  expect(tjev_gdn_mega2_fwd_normed(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                   (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, fake(24),
                                   (const float*)fake(25), -1.f, fake(7), fake(26), (float*)fake(8), nullptr, nullptr,
                                   ws, 0),
         TJEV_GDN_EINVAL, "fwd_normed negative eps");
  expect(tjev_gdn_mega2_bwd_normed(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                   (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, (const float*)f[8],
                                   fake(7), fake(24), (const float*)fake(25), 1e-6f, fake(9), nullptr, fake(10),
                                   fake(11), fake(12), (float*)fake(13), (float*)fake(14), nullptr, nullptr, nullptr,
                                   fake(26), (float*)fake(27), ws, 0),
         TJEV_GDN_EWORKSPACE, "bwd_normed");
  expect(tjev_gdn_mega2_bwd_normed(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                   (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, (const float*)f[8],
                                   nullptr, fake(24), (const float*)fake(25), 1e-6f, fake(9), nullptr, fake(10),
                                   fake(11), fake(12), (float*)fake(13), (float*)fake(14), nullptr, nullptr, nullptr,
                                   fake(26), nullptr, ws, 0),
         TJEV_GDN_EINVAL, "bwd_normed null out");
  if (tjev_gdn_workspace_bytes_normed(&p, 1) <= tjev_gdn_workspace_bytes(&p, 1)) {
    std::printf("MISMATCH workspace_bytes_normed\n");
    ++g_bad;
  }
  expect(tjev_gdn_mega2_bwd_cont(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                 (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, (const float*)f[8], f[9],
                                 (const float*)fake(22), fake(10), fake(11), fake(12), (float*)fake(13),
                                 (float*)fake(14), nullptr, nullptr, nullptr, ws, 0),
         TJEV_GDN_EWORKSPACE, "bwd_cont final-state gradient on a ragged length (accepted; no workspace)");
  expect(tjev_gdn_mega2_bwd_cont(&p, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                 (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, (const float*)f[8], f[9],
                                 nullptr, fake(10), fake(11), fake(12), (float*)fake(13), (float*)fake(14), nullptr,
                                 (float*)fake(24), nullptr, ws, 0),
         TJEV_GDN_EINVAL, "bwd_cont initial-state gradient without the state");
  {
    tjev_gdn_params big = params(4, 4096, 16, 128, 16, 4, 128);
    expect(tjev_gdn_mega2_fwd_cont_noalloc(&big, nullptr, f[0], f[1], f[2], (const float*)f[3], (const float*)f[4],
                                           (const float*)f[5], (const int32_t*)f[6], nullptr, nullptr, fake(7),
                                           (float*)fake(8), nullptr, nullptr),
           TJEV_GDN_EWORKSPACE, "noalloc beyond the scratch");
  }
  // the v2 operator
  {
    tjev_gdn_params v = params(2, 300, 2, 16, 4, 0, 16);
    expect(tjev_gdn_v2_fwd(&v, nullptr, f[0], f[1], f[2], f[3], f[4], (const int32_t*)f[5], fake(6), (float*)fake(7),
                           ws, 0),
           TJEV_GDN_EWORKSPACE, "v2 fwd no workspace");
    expect(tjev_gdn_v2_fwd(&p, nullptr, f[0], f[1], f[2], f[3], f[4], (const int32_t*)f[5], fake(6), (float*)fake(7),
                           ws, 0),
           TJEV_GDN_EINVAL, "v2 with taps");
    expect(tjev_gdn_v2_bwd_cont(&v, nullptr, f[0], f[1], f[2], f[3], f[4], (const int32_t*)f[5], nullptr,
                                (const float*)f[7], f[8], nullptr, fake(9), fake(10), fake(11), fake(12), fake(13),
                                (float*)fake(14), ws, 0),
           TJEV_GDN_EINVAL, "v2 bwd_cont state gradient without the state");
  }
  // the decode step
  {
    tjev_gdn_params d = params(4, 1, 2, 16, 4, 4, 64);
    void* b[11];
    for (int i = 0; i < 11; ++i) b[i] = fake(50 + i);
    tjev_gdn_params two = d;
    two.length = 2;
    expect(tjev_gdn_decode_step(&two, nullptr, b[0], b[1], b[2], (const float*)b[3], (const float*)b[4],
                                (const float*)b[5], b[6], (const float*)b[7], b[8], b[9], (float*)b[10]),
           TJEV_GDN_EINVAL, "decode: two tokens");
    expect(tjev_gdn_decode_step(&d, nullptr, b[0], b[1], b[2], (const float*)b[3], (const float*)b[4],
                                (const float*)b[5], b[6], (const float*)b[7], b[8], b[6], (float*)b[10]),
           TJEV_GDN_EINVAL, "decode: aliased history");
    expect(tjev_gdn_decode_step(&d, nullptr, odd(50), b[1], b[2], (const float*)b[3], (const float*)b[4],
                                (const float*)b[5], b[6], (const float*)b[7], b[8], b[9], (float*)b[10]),
           TJEV_GDN_EINVAL, "decode: misaligned qkv");
  }
  // the gated RMSNorm
  {
    tjev_gdn_norm_params n;
    n.tokens = 100;
    n.heads = 4;
    n.dim = 128;
    n.dtype = TJEV_GDN_BF16;
    n.eps = 1e-6f;
    expect(tjev_gdn_gated_rmsnorm_fwd(&n, nullptr, nullptr, f[1], (const float*)f[2], nullptr, fake(3)),
           TJEV_GDN_EINVAL, "norm null x");
    expect(tjev_gdn_gated_rmsnorm_fwd(&n, nullptr, odd(0), f[1], (const float*)f[2], nullptr, fake(3)),
           TJEV_GDN_EINVAL, "norm misaligned x");
    expect(tjev_gdn_gated_rmsnorm_bwd(&n, nullptr, f[0], f[1], (const float*)f[2], nullptr, f[3], fake(4), fake(5),
                                      (float*)fake(6), nullptr, 0),
           TJEV_GDN_EWORKSPACE, "norm weight gradient without workspace");
    tjev_gdn_norm_params bad = n;
    bad.dim = 48;
    expect(tjev_gdn_gated_rmsnorm_fwd(&bad, nullptr, f[0], f[1], (const float*)f[2], nullptr, fake(3)),
           TJEV_GDN_EUNSUPPORTED, "norm dim");
    tjev_gdn_norm_params empty = n;
    empty.tokens = 0;
    expect(tjev_gdn_gated_rmsnorm_fwd(&empty, nullptr, nullptr, nullptr, (const float*)f[2], nullptr, nullptr), 0,
           "norm of no tokens");
  }
  // names, versions, profiling with nothing recorded
  for (int k = -1; k <= TJEV_GDN_KERNELS; ++k)
    if (!tjev_gdn_kernel_name(k)) ++g_bad;
  float ms[TJEV_GDN_KERNELS];
  int launches[TJEV_GDN_KERNELS];
  expect(tjev_gdn_profile_begin(), 0, "profile begin");
  expect(tjev_gdn_profile_end(ms, launches, TJEV_GDN_KERNELS), 0, "profile end");
  std::printf("abi driver: %d mismatches\n", g_bad);
  return g_bad;
}
