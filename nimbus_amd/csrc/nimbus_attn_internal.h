// Constants shared by the kernels and the C ABI in include/nimbus_attn.h.
#pragma once

#include "nimbus_attn.h"

namespace nimbus {

constexpr int kPrefillTile = NIMBUS_PREFILL_TILE;          // query positions per tile-table entry

}  // namespace nimbus
