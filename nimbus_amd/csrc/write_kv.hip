// KV slot write for gfx950: scatter new K/V token rows into the paged caches.
//
// Replaces nimbus/kernels/reference.py:14-23 (two index_copy_ calls through
// the flat [num_blocks * block_size, KV, D] view of each cache) with one
// launch that moves both K and V. Thread i copies one 16-byte piece of one
// (token, kv head) row of K and the same piece of V; a wave covers whole
// rows, so reads of k/v and writes into the slot are coalesced. The copy is
// bitwise (no conversion), which makes the result bit-exact on unique slots.
// A scalar variant handles sources whose strides break 16-byte alignment.
#include "common.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

struct WriteKVArgs {
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* kc;
  uint16_t* vc;
  const int64_t* slots;
  int64_t n_tokens;
  int64_t k_st, k_sh, v_st, v_sh;
  int64_t num_slots;
  int32_t kv, d;
};

// PIECES: 16-byte pieces per head row (8 at head_dim 64, 16 at 128; 0 for any
// other head_dim, read from the arguments). The host launches it only when
// the piece count fits 32 bits, so the index arithmetic is 32-bit (a 64-bit
// divide per piece cost more than the copy).
template <int PIECES>
__global__ __launch_bounds__(256) void write_kv_vec_kernel(WriteKVArgs a) {
  const uint32_t pieces = PIECES ? PIECES : a.d / 8;
  const uint32_t per_token = static_cast<uint32_t>(a.kv) * pieces;
  const uint32_t total = static_cast<uint32_t>(a.n_tokens) * per_token;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < total; i += gridDim.x * blockDim.x) {
    const uint32_t t32 = i / per_token;
    const uint32_t rem = i - t32 * per_token;
    const int h = static_cast<int>(rem / pieces);
    const int c = static_cast<int>(rem - h * pieces);
    const int64_t t = t32;
    const int64_t slot = a.slots[t];
    if (slot < 0 || slot >= a.num_slots) continue;
    const u32x4 kv = *reinterpret_cast<const u32x4*>(a.k + t * a.k_st + h * a.k_sh + 8 * c);
    const u32x4 vv = *reinterpret_cast<const u32x4*>(a.v + t * a.v_st + h * a.v_sh + 8 * c);
    const int64_t dst = (slot * a.kv + h) * a.d + 8 * c;
    *reinterpret_cast<u32x4*>(a.kc + dst) = kv;
    *reinterpret_cast<u32x4*>(a.vc + dst) = vv;
  }
}

__global__ __launch_bounds__(256) void write_kv_scalar_kernel(WriteKVArgs a) {
  const int64_t per_token = static_cast<int64_t>(a.kv) * a.d;
  const int64_t total = a.n_tokens * per_token;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / per_token;
    const int rem = static_cast<int>(i - t * per_token);
    const int h = rem / a.d;
    const int e = rem - h * a.d;
    const int64_t slot = a.slots[t];
    if (slot < 0 || slot >= a.num_slots) continue;
    const int64_t dst = (slot * a.kv + h) * a.d + e;
    a.kc[dst] = a.k[t * a.k_st + h * a.k_sh + e];
    a.vc[dst] = a.v[t * a.v_st + h * a.v_sh + e];
  }
}

}  // namespace nimbus

using namespace nimbus;

extern "C" int nimbus_attn_abi_version(void) { return NIMBUS_ATTN_ABI_VERSION; }

extern "C" const char* nimbus_attn_error_string(int code) {
  switch (code) {
    case NIMBUS_OK:
      return "ok";
    case NIMBUS_ERR_INVALID:
      return "invalid argument (inconsistent sizes or null pointer)";
    case NIMBUS_ERR_UNSUPPORTED:
      return "unsupported shape or dtype (block_size must be 16, head_dim 64 or 128, dtype fp16 or bf16)";
    case NIMBUS_ERR_ALIGNMENT:
      return "a base pointer or stride breaks 16-byte vector access";
    case NIMBUS_ERR_WORKSPACE:
      return "workspace missing or smaller than the entry point's *_workspace_bytes()";
    case NIMBUS_ERR_SCRATCH:
      return "the call needs more workspace than nimbus_paged_decode_noalloc's scratch "
             "(NIMBUS_NOALLOC_SCRATCH_BYTES); use nimbus_paged_decode with a workspace";
    default:
      return code > 0 ? hipGetErrorString(static_cast<hipError_t>(code)) : "unknown error";
  }
}

extern "C" int nimbus_write_kv(const void* k, const void* v, void* k_cache, void* v_cache,
                               const int64_t* slot_mapping, int64_t num_tokens, int32_t num_kv_heads,
                               int32_t head_dim, int64_t k_stride_token, int64_t k_stride_head,
                               int64_t v_stride_token, int64_t v_stride_head, int64_t num_slots, int32_t dtype,
                               void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (num_tokens == 0) return NIMBUS_OK;
  if (!k || !v || !k_cache || !v_cache || !slot_mapping) return NIMBUS_ERR_INVALID;
  WriteKVArgs a;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.kc = static_cast<uint16_t*>(k_cache);
  a.vc = static_cast<uint16_t*>(v_cache);
  a.slots = slot_mapping;
  a.n_tokens = num_tokens;
  a.k_st = k_stride_token;
  a.k_sh = k_stride_head;
  a.v_st = v_stride_token;
  a.v_sh = v_stride_head;
  a.num_slots = num_slots;
  a.kv = num_kv_heads;
  a.d = head_dim;
  const bool vec = head_dim % 8 == 0 && (k_stride_token | k_stride_head | v_stride_token | v_stride_head) % 8 == 0 &&
                   ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
                     reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) % 16) == 0;
  const int64_t work = num_tokens * num_kv_heads * (vec ? head_dim / 8 : head_dim);
  int64_t blocks = (work + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (vec && work < (int64_t{1} << 31)) {
    if (head_dim == 128) hipLaunchKernelGGL(write_kv_vec_kernel<16>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
    else if (head_dim == 64) hipLaunchKernelGGL(write_kv_vec_kernel<8>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
    else hipLaunchKernelGGL(write_kv_vec_kernel<0>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL(write_kv_scalar_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}
