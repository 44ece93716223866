// Kernel tables without kernels, for the host-only AddressSanitizer build of the C ABI
// (tests/test_asan_host.py): every (chunk, head dim) of gdn_shapes.def has a table, so the
// validation paths run exactly as in the library; its launch functions are null and the
// driver never gets that far (every call it makes fails validation or finds no workspace).
#include "../../tjev_amd/csrc/gdn_launch.h"

namespace gdn {
#define GDN_SHAPE(c, d)                          \
  const ShapeTable* table_##c##_##d() {          \
    static const ShapeTable t = [] {             \
      ShapeTable s{};                            \
      s.C = c;                                   \
      s.D = d;                                   \
      return s;                                  \
    }();                                         \
    return &t;                                   \
  }
#include "../../tjev_amd/csrc/gdn_shapes.def"
#undef GDN_SHAPE
}  // namespace gdn
