// Runtime specialization of elementwise programs (jit.hip).
#pragma once

#include "common.h"

namespace pdh {

enum class JitKind { MapChain, Contract };

bool jit_enabled();
// fns[0] (and, for map chains, fns[1]: the one-element-per-lane variant) of
// the kernel specialized for program p and element type dt; false when the
// interpreter kernels must run it (disabled, or the compile failed).
bool jit_get(JitKind kind, const pdh_ew_program& p, int dt, hipFunction_t fns[2]);
void jit_count_launch();

}  // namespace pdh
