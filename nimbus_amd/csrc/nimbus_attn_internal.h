// Constants shared by the kernels and the C ABI in include/nimbus_attn.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nimbus_attn.h"

namespace nimbus {

constexpr int kPrefillTile = NIMBUS_PREFILL_TILE;          // query positions per tile-table entry

// CU count of the current device (asked of the runtime once per device);
// 0 or a hipError_t.
int device_cus(int64_t* cus);

// ---- paged attention for page sizes other than 16 and head dims other than
// 64 and 128 (paged_general.hip)
constexpr int kGenMaxHeadDim = 256;
constexpr int kGenMaxChunkElems = 2048;  // query heads x head dim per workgroup
constexpr int kGenMaxHeads = 64;         // query heads per workgroup

struct AttnGeneralArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;  // per query row (token), per head
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t c_sb, c_st, c_sh;
  const int32_t* bt;
  int64_t bt_sb;
  int32_t bt_width, num_blocks, bs;
  const int32_t* ctx;
  int32_t nq, max_ctx;              // decode and verify rows: b * nq + j
  const int32_t* qstart;            // prefill rows: positions of tile-table entries
  const int32_t* prog_seq;
  const int32_t* prog_m;
  int32_t tile_pos;                 // query positions per tile-table entry
  uint16_t* out;
  int64_t o_st, o_sh;
  int32_t H, G, KV, D;
  int32_t gc, nchunks;              // set by the launchers
  float scale_log2;
};

// Whether a shape takes the general kernel, and whether it can.
bool general_shape(int32_t head_dim, int32_t block_size);
int general_check(int32_t head_dim, int32_t block_size);
int launch_general_decode(const AttnGeneralArgs& a, int64_t batch, int dtype, hipStream_t s);
int launch_general_prefill(const AttnGeneralArgs& a, int64_t num_programs, int dtype, hipStream_t s);

}  // namespace nimbus
