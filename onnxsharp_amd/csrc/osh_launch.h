// osh_launch.h -- internal launchers shared between the entry-point files.
#pragma once

#include "osh_common.h"

namespace osh {

struct IgemmArgs;

// Launches the MFMA implicit-GEMM tile over zcount z-slices (B_DENSE or B_IM2COL).
osh_status launch_igemm(const IgemmArgs &a, int zcount, int bmode, int act, hipStream_t st);

}  // namespace osh
