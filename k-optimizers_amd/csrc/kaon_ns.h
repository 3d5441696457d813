// kaon_ns.h -- AdaMuon's Newton-Schulz stage (kaon_ns.hip), called by the
// AdaMuon step in kaon_step.hip.
#pragma once

#include <hip/hip_runtime.h>

#include "kaon_amd.h"

// Runs, for every tensor of the plan: the scaled (and, when R > C,
// transposed) bf16 iterate X = M / (||M|| + 1e-7) from the momentum buffer M
// in the workspace, `steps` quintic iterations, and the orthogonal factor O
// written back over M in the [R, C] orientation.  Returns 0 or a HIP error
// code (kaon_last_error set).
int kaon_ns_run(const KaonLaunch& L, int steps, hipStream_t stream);
