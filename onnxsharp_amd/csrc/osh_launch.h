// osh_launch.h -- internal launchers shared between the entry-point files.
#pragma once

#include "osh_common.h"

namespace osh {

struct IgemmArgs;

// Launches the MFMA implicit-GEMM tile over zcount z-slices (B_DENSE or B_IM2COL).
osh_status launch_igemm(const IgemmArgs &a, int zcount, int bmode, int act, hipStream_t st);

// Whether d_w holds weights this library packed for the 1x1 conv p in the
// pointwise LDS-tile layout ([ceil(M/16)][C/16][64 lanes][4 steps], then the
// raw [M][C] operand).
bool packed_for_pointwise_tiles(const osh_conv_params *p, const void *d_w);

}  // namespace osh
