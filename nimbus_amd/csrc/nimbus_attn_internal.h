// Constants shared by the kernels and the C ABI in include/nimbus_attn.h.
#pragma once

#include "nimbus_attn.h"

namespace nimbus {

constexpr int kPrefillTile = NIMBUS_PREFILL_TILE;          // query positions per tile-table entry

// CU count of the current device (asked of the runtime once per device);
// 0 or a hipError_t.
int device_cus(int64_t* cus);

}  // namespace nimbus
