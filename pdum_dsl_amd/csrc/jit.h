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
// lay: the fp32 contraction's operand layouts (contract_split_body's LAY);
// red: its row-partial reduction (ContractArgs::rowred, -1 for none).
bool jit_get(JitKind kind, const pdh_ew_program& p, int dt, hipFunction_t fns[2], int lay = 0, int red = -1);
// The row-reduce kernels specialized for (summand, epilogue): fns[0] one wave
// per output, fns[1] the column variant; or false.
bool jit_get_reduce(const pdh_ew_program& ps, const pdh_ew_program& pe, int dt, hipFunction_t fns[2]);
// The fp32 contraction with operand prologues (pa / pb null: read as a view),
// specialized: fns[0] the 128 x 128-tile (or fp32-mode-0 VALU) kernel, fns[1]
// the 64 x 64-tile one; or false.
bool jit_get_pro(const pdh_ew_program& pe, const pdh_ew_program* pa, const pdh_ew_program* pb, hipFunction_t fns[2],
                 int lay, int dt);
void jit_count_launch();
// How fp32 contractions run: 0 VALU fma; 1, 3 or 6 bf16 MFMA products per term
// (pdh_contract_set_f32_mode).
int f32_contract_mode();

}  // namespace pdh
