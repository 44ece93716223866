// Host-side launch table shared by the instantiation units and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "gdn_args.h"

namespace gdn {

// Kernel ids of the two sequences (the per-kernel timing slots of tjev_gdn_profile_*).
enum KernelId : int {
  K_PREP_FWD = 0, K_CHUNK_FWD, K_SCAN_FWD, K_OUT,
  K_PREP_BWD, K_CHUNK_BWD, K_BWD_LOCAL, K_SCAN_BWD, K_BWD_GRADS, K_POST, K_REDUCE,
  K_NORM_FWD, K_NORM_BWD, K_NORM_REDUCE,
  K_FINAL_STATE, K_DECODE,
  K_COUNT
};

// Optional timing hook: called with end = 0 just before and end = 1 just after each launch.
struct Timer {
  void (*mark)(void* self, int kernel, int end, hipStream_t stream);
  void* self;
};

// runs the forward (backward = 0) or backward (1) kernel sequence on the stream
typedef hipError_t (*GdnFn)(const GdnArgs&, hipStream_t, int backward, const Timer* timer);

struct ShapeTable {
  int C, D;
  GdnFn fn[4][2][2];       // [precision][io dtype][gate dtype]
  GdnFn fnv2[4][2][2][2];  // the v2 operator: [precision][io dtype][q/k dtype][gate dtype]
};

// Shared by the C ABI's units (defined in gdn_api.hip): record the message of a nonzero status
// for tjev_gdn_last_error(), and the timing hook while profiling is on (else null).
int fail(int status, const char* msg);
const Timer* active_timer();

#define GDN_SHAPE(c, d) const ShapeTable* table_##c##_##d();
#include "gdn_shapes.def"
#undef GDN_SHAPE

}  // namespace gdn
