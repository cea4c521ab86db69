// gg_resources.cpp -- per-kernel register and LDS figures of the compiled kernels.
//
// The table comes from the compiler's resource-usage report for
// gg_kernels.hip (VGPRs, AGPRs, SGPRs, scratch, waves per SIMD, LDS), which the
// build writes to gg_resources_table.inc.  hipFuncGetAttributes has no AGPR
// field, so query_occupancy takes the register split from here.
#include <stddef.h>

namespace {

struct ResourceRow {
  int kind;  // GGK_KERNEL_GROUPED or GGK_KERNEL_SINGLE
  int variant;
  int path;
  int vgprs;
  int agprs;
  int sgprs;
  int scratch;
  int waves_per_simd;
  int lds;
};

const ResourceRow kRows[] = {
#include "gg_resources_table.inc"
    {-1, -1, -1, 0, 0, 0, 0, 0, 0},
};

}  // namespace

extern "C" int gg_compiler_resources(int kind, int variant, int path, int* vgprs, int* agprs, int* sgprs,
                                     int* scratch, int* waves_per_simd, int* lds) {
  for (size_t i = 0; i < sizeof(kRows) / sizeof(kRows[0]); ++i) {
    const ResourceRow& r = kRows[i];
    if (r.kind == kind && r.variant == variant && r.path == path) {
      *vgprs = r.vgprs;
      *agprs = r.agprs;
      *sgprs = r.sgprs;
      *scratch = r.scratch;
      *waves_per_simd = r.waves_per_simd;
      *lds = r.lds;
      return 0;
    }
  }
  return -1;
}
