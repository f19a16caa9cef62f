// Runtime specialization of elementwise programs (jit.hip).
#pragma once

#include "common.h"

namespace pdh {

enum class JitKind { MapChain, Contract };

bool jit_enabled();
// fns[0] (and fns[1]: the one-element-per-lane map chain; the 64 x 64-tile
// contraction) of
// the kernel specialized for program p and element type dt; false when the
// interpreter kernels must run it (disabled, or the compile failed).
bool jit_get(JitKind kind, const pdh_ew_program& p, int dt, hipFunction_t fns[2]);
// The row-reduce kernel specialized for (summand, epilogue), or false.
bool jit_get_reduce(const pdh_ew_program& ps, const pdh_ew_program& pe, int dt, hipFunction_t* fn);
void jit_count_launch();

}  // namespace pdh
