// Rotary embedding and SiLU-gated product of the Llama decoder for gfx950.
//
// nimbus_rope replaces Rotary.forward (nimbus/model/llama.py:37-57): for
// token t at position p, every head's pairs (i, i + D/2) become
//   out_i       = x_i c_i - x_{i+D/2} s_i
//   out_{i+D/2} = x_{i+D/2} c_{i+D/2} + x_i s_{i+D/2}
// with c = dtype(cos[p]), s = dtype(sin[p]) (the fp32 tables of llama.py:
// 43-47 cast to the model dtype). Each product and the sum are rounded to
// the model dtype, as the reference's separate multiplies and add are, so
// the result is the reference's bit for bit. It runs in place on the q and k
// parts of the fused qkv projection (one launch for both).
//
// nimbus_rope_write_kv is nimbus_rope on the q and k heads of the fused qkv
// rows followed by nimbus_write_kv of their k and v heads (the model's
// Attention.forward then AttentionBackend.forward, nimbus/model/llama.py:
// 88-98 and nimbus/model/attention.py:78), in one launch and with the same
// results bit for bit.
//
// nimbus_silu_mul replaces MLP.forward's F.silu(gate) * up
// (nimbus/model/llama.py:93-103): silu in fp32 rounded to the model dtype,
// then the product rounded again.
//
// nimbus_greedy_step is one link of DecodeGraphs.greedy_chain
// (nimbus/cuda_graph.py:92-116) on the device: per row, the argmax of the
// logits (first index among equal maxima, as torch.argmax) becomes the next
// input token and is recorded, and the row's position, context length and
// cache slot advance.
#include "common.h"
#include "nimbus_attn_internal.h"
#include "silu.h"

namespace nimbus {

struct RopeArgs {
  uint16_t* x;
  int64_t sx;        // elements between tokens
  const int64_t* pos;
  const float* cos;
  const float* sin;
  int64_t st;        // elements between table rows
  int32_t tokens, heads, d, max_pos;
};

template <int DT>
__device__ __forceinline__ float rnd(float v) {
  return Elem<DT>::to_f32(Elem<DT>::from_f32(v));
}

// Rotates 8 pairs of one head: lo holds x[i0 .. i0 + 8), hi holds
// x[i0 + D/2 .. + 8), cr / sr point at the position's table rows.
template <int DT>
__device__ __forceinline__ void rope_pairs(u32x4& lo, u32x4& hi, const float* cr, const float* sr, int i0, int half) {
  // The products are rounded before the add; a fused multiply-add would skip
  // that rounding (hipcc contracts by default).
#pragma clang fp contract(off)
  // The table rows' 8 entries at i0 and at i0 + D/2, as 16-byte loads.
  float c_lo[8], s_lo[8], c_hi[8], s_hi[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    *reinterpret_cast<f32x4*>(&c_lo[4 * h]) = *reinterpret_cast<const f32x4*>(cr + i0 + 4 * h);
    *reinterpret_cast<f32x4*>(&s_lo[4 * h]) = *reinterpret_cast<const f32x4*>(sr + i0 + 4 * h);
    *reinterpret_cast<f32x4*>(&c_hi[4 * h]) = *reinterpret_cast<const f32x4*>(cr + half + i0 + 4 * h);
    *reinterpret_cast<f32x4*>(&s_hi[4 * h]) = *reinterpret_cast<const f32x4*>(sr + half + i0 + 4 * h);
  }
  u32x4 olo, ohi;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t out_lo[2], out_hi[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int j = 2 * e + b;
      const float xl = Elem<DT>::to_f32(static_cast<uint16_t>(lo[e] >> (16 * b)));
      const float xh = Elem<DT>::to_f32(static_cast<uint16_t>(hi[e] >> (16 * b)));
      const float cl = rnd<DT>(c_lo[j]), sl = rnd<DT>(s_lo[j]);
      const float ch = rnd<DT>(c_hi[j]), sh = rnd<DT>(s_hi[j]);
      // x * cos + rotate_half(x) * sin, rotate_half(x) = cat(-x_hi, x_lo)
      out_lo[b] = Elem<DT>::from_f32(rnd<DT>(xl * cl) + rnd<DT>(-xh * sl));
      out_hi[b] = Elem<DT>::from_f32(rnd<DT>(xh * ch) + rnd<DT>(xl * sh));
    }
    olo[e] = pack2(out_lo[0], out_lo[1]);
    ohi[e] = pack2(out_hi[0], out_hi[1]);
  }
  lo = olo;
  hi = ohi;
}

// One thread per (token, head, 8 consecutive i < D/2): 16-byte loads of x at
// i and i + D/2.
template <int DT>
__global__ __launch_bounds__(256) void rope_kernel(RopeArgs a) {
  const int half = a.d / 2;
  const int per_head = half / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.tokens) * a.heads * per_head;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % per_head);
  const int h = static_cast<int>((idx / per_head) % a.heads);
  const int64_t t = idx / (static_cast<int64_t>(per_head) * a.heads);
  const int64_t p = a.pos[t];
  if (p < 0 || p >= a.max_pos) return;  // no table row: left as is
  const int i0 = 8 * c;
  uint16_t* row = a.x + t * a.sx + static_cast<int64_t>(h) * a.d;
  u32x4 lo = *reinterpret_cast<const u32x4*>(row + i0);
  u32x4 hi = *reinterpret_cast<const u32x4*>(row + half + i0);
  rope_pairs<DT>(lo, hi, a.cos + p * a.st, a.sin + p * a.st, i0, half);
  *reinterpret_cast<u32x4*>(row + i0) = lo;
  *reinterpret_cast<u32x4*>(row + half + i0) = hi;
}

struct RopeWriteArgs {
  RopeArgs r;  // x = the qkv rows, heads = q heads + kv heads (the rotated ones)
  int32_t q_heads, kv_heads;
  uint16_t* kc;
  uint16_t* vc;
  const int64_t* slots;
  int64_t num_slots;
};

// nimbus_rope over the q and k heads, then nimbus_write_kv of the k and v
// heads, in one launch: one thread per (token, q / k head, 8 pairs). A k
// head's thread also stores its rotated 16-byte pieces into the K cache
// slot and copies the same two pieces of the token's v head into the V
// cache slot.
template <int DT>
__global__ __launch_bounds__(256) void rope_write_kv_kernel(RopeWriteArgs w) {
  const RopeArgs& a = w.r;
  const int half = a.d / 2;
  const int per_head = half / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(a.tokens) * a.heads * per_head;
  if (idx >= total) return;
  const int c = static_cast<int>(idx % per_head);
  const int h = static_cast<int>((idx / per_head) % a.heads);
  const int64_t t = idx / (static_cast<int64_t>(per_head) * a.heads);
  const int64_t p = a.pos[t];
  const bool rotate = p >= 0 && p < a.max_pos;  // no table row: left as is
  const int i0 = 8 * c;
  uint16_t* row = a.x + t * a.sx + static_cast<int64_t>(h) * a.d;
  u32x4 lo = *reinterpret_cast<const u32x4*>(row + i0);
  u32x4 hi = *reinterpret_cast<const u32x4*>(row + half + i0);
  if (rotate) {
    rope_pairs<DT>(lo, hi, a.cos + p * a.st, a.sin + p * a.st, i0, half);
    *reinterpret_cast<u32x4*>(row + i0) = lo;
    *reinterpret_cast<u32x4*>(row + half + i0) = hi;
  }
  const int kh = h - w.q_heads;
  if (kh < 0) return;
  const int64_t slot = w.slots[t];
  if (slot < 0 || slot >= w.num_slots) return;
  const int64_t dst = (slot * w.kv_heads + kh) * a.d;
  *reinterpret_cast<u32x4*>(w.kc + dst + i0) = lo;
  *reinterpret_cast<u32x4*>(w.kc + dst + half + i0) = hi;
  const uint16_t* vrow = row + static_cast<int64_t>(w.kv_heads) * a.d;  // v head kh follows the k heads
  *reinterpret_cast<u32x4*>(w.vc + dst + i0) = *reinterpret_cast<const u32x4*>(vrow + i0);
  *reinterpret_cast<u32x4*>(w.vc + dst + half + i0) = *reinterpret_cast<const u32x4*>(vrow + half + i0);
}

struct SiluArgs {
  const uint16_t* x;
  int64_t sx;
  uint16_t* out;
  int64_t so;
  int32_t rows, cols;
};

// One thread per 8 consecutive outputs of a row.
template <int DT>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluArgs a) {
  const int per_row = a.cols / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(a.rows) * per_row) return;
  const int64_t r = idx / per_row;
  const int c = static_cast<int>(idx % per_row) * 8;
  const uint16_t* xr = a.x + r * a.sx;
  const u32x4 g = *reinterpret_cast<const u32x4*>(xr + c);
  const u32x4 u = *reinterpret_cast<const u32x4*>(xr + a.cols + c);
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint16_t v[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const float gv = Elem<DT>::to_f32(static_cast<uint16_t>(g[e] >> (16 * b)));
      const float uv = Elem<DT>::to_f32(static_cast<uint16_t>(u[e] >> (16 * b)));
      v[b] = silu_mul_value<DT>(gv, uv);
    }
    o[e] = pack2(v[0], v[1]);
  }
  *reinterpret_cast<u32x4*>(a.out + r * a.so + c) = o;
}

struct GreedyArgs {
  const float* logits;
  int64_t sl;
  int32_t rows, vocab;
  int64_t* input_ids;
  int64_t* positions;
  int32_t* ctx;
  int64_t* slots;
  const int32_t* tables;
  int64_t bt_stride;
  int32_t bt_width, block_size;
  const int32_t* active;
  const int32_t* ctx_start;
  int64_t* tokens;
  int32_t max_steps;
  int64_t scratch_slot;
};

// (value, index) order of the argmax: larger value, then smaller index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

constexpr int kGreedyThreads = 1024;

__device__ __forceinline__ void consider(float v, int i, float& bv, int& bi) {
  if (better(v, i, bv, bi)) {
    bv = v;
    bi = i;
  }
}

// One 1024-thread workgroup per row. With 16-byte aligned rows, each thread
// reads float4 pieces 1024 apart, four loads in flight before any compare.
__global__ __launch_bounds__(kGreedyThreads) void greedy_step_kernel(GreedyArgs a) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float* lr = a.logits + static_cast<int64_t>(row) * a.sl;
  float bv = -INFINITY;
  int bi = a.vocab;
  const bool vec = (a.sl % 4 == 0) && (reinterpret_cast<uintptr_t>(a.logits) % 16 == 0);
  const int nvec = vec ? a.vocab / 4 : 0;
  const f32x4* lv = reinterpret_cast<const f32x4*>(lr);
  int i = tid;
  for (; i + 3 * kGreedyThreads < nvec; i += 4 * kGreedyThreads) {
    f32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = lv[i + u * kGreedyThreads];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
#pragma unroll
      for (int e = 0; e < 4; ++e) consider(v[u][e], 4 * (i + u * kGreedyThreads) + e, bv, bi);
    }
  }
  for (; i < nvec; i += kGreedyThreads) {
    const f32x4 v = lv[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) consider(v[e], 4 * i + e, bv, bi);
  }
  for (int j = 4 * nvec + tid; j < a.vocab; j += kGreedyThreads) consider(lr[j], j, bv, bi);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    consider(ov, oi, bv, bi);
  }
  __shared__ float sv[kGreedyThreads / 64];
  __shared__ int si[kGreedyThreads / 64];
  if (tid % 64 == 0) {
    sv[tid / 64] = bv;
    si[tid / 64] = bi;
  }
  __syncthreads();
  if (tid != 0) return;
  for (int w = 1; w < kGreedyThreads / 64; ++w) consider(sv[w], si[w], bv, bi);
  const int64_t tok = bi < a.vocab ? bi : 0;  // a row of NaNs picks token 0
  a.input_ids[row] = tok;
  if (!a.active[row]) return;
  const int k = a.ctx[row] - a.ctx_start[row];
  if (k >= 0 && k < a.max_steps) a.tokens[static_cast<int64_t>(row) * a.max_steps + k] = tok;
  const int64_t p = a.positions[row] + 1;
  a.positions[row] = p;
  a.ctx[row] += 1;
  const int64_t page = p / a.block_size;
  a.slots[row] = page < a.bt_width
                     ? static_cast<int64_t>(a.tables[row * a.bt_stride + page]) * a.block_size + p % a.block_size
                     : a.scratch_slot;
}

}  // namespace nimbus

using namespace nimbus;

extern "C" int nimbus_greedy_step(const float* logits, int64_t logits_stride, int32_t rows, int32_t vocab,
                                  int64_t* input_ids, int64_t* positions, int32_t* context_lens, int64_t* slots,
                                  const int32_t* block_tables, int64_t bt_stride, int32_t bt_width,
                                  int32_t block_size, const int32_t* active, const int32_t* ctx_start,
                                  int64_t* tokens, int32_t max_steps, int64_t scratch_slot, void* stream) {
  if (rows < 0 || vocab <= 0 || block_size <= 0 || bt_width <= 0 || max_steps < 0) return NIMBUS_ERR_INVALID;
  if (rows == 0) return NIMBUS_OK;
  if (!logits || !input_ids || !positions || !context_lens || !slots || !block_tables || !active || !ctx_start ||
      (max_steps > 0 && !tokens))
    return NIMBUS_ERR_INVALID;
  if (logits_stride < vocab || bt_stride < bt_width) return NIMBUS_ERR_INVALID;
  GreedyArgs a;
  a.logits = logits;
  a.sl = logits_stride;
  a.rows = rows;
  a.vocab = vocab;
  a.input_ids = input_ids;
  a.positions = positions;
  a.ctx = context_lens;
  a.slots = slots;
  a.tables = block_tables;
  a.bt_stride = bt_stride;
  a.bt_width = bt_width;
  a.block_size = block_size;
  a.active = active;
  a.ctx_start = ctx_start;
  a.tokens = tokens;
  a.max_steps = max_steps;
  a.scratch_slot = scratch_slot;
  hipLaunchKernelGGL(greedy_step_kernel, dim3(rows), dim3(kGreedyThreads), 0, static_cast<hipStream_t>(stream), a);
  return static_cast<int>(hipGetLastError());
}

extern "C" int nimbus_rope(void* x, int64_t x_stride, int64_t num_tokens, int32_t num_heads, int32_t head_dim,
                           const int64_t* positions, const float* cos_table, const float* sin_table,
                           int64_t table_stride, int32_t max_position, int32_t dtype, void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || head_dim <= 0 || max_position <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (head_dim % 16 != 0 || num_tokens > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
  if (num_tokens == 0) return NIMBUS_OK;
  if (!x || !positions || !cos_table || !sin_table) return NIMBUS_ERR_INVALID;
  if (x_stride < static_cast<int64_t>(num_heads) * head_dim || table_stride < head_dim) return NIMBUS_ERR_INVALID;
  if (x_stride % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0) return NIMBUS_ERR_ALIGNMENT;
  if (table_stride % 4 != 0 ||
      (reinterpret_cast<uintptr_t>(cos_table) | reinterpret_cast<uintptr_t>(sin_table)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  RopeArgs a;
  a.x = static_cast<uint16_t*>(x);
  a.sx = x_stride;
  a.pos = positions;
  a.cos = cos_table;
  a.sin = sin_table;
  a.st = table_stride;
  a.tokens = static_cast<int32_t>(num_tokens);
  a.heads = num_heads;
  a.d = head_dim;
  a.max_pos = max_position;
  const int64_t threads = num_tokens * num_heads * (head_dim / 16);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kFloat16) {
    hipLaunchKernelGGL((rope_kernel<kFloat16>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((rope_kernel<kBFloat16>), grid, dim3(256), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int nimbus_rope_write_kv(void* qkv, int64_t qkv_stride, int64_t num_tokens, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, const int64_t* positions,
                                    const float* cos_table, const float* sin_table, int64_t table_stride,
                                    int32_t max_position, void* k_cache, void* v_cache, const int64_t* slot_mapping,
                                    int64_t num_slots, int32_t dtype, void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_position <= 0 ||
      num_slots < 0)
    return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (head_dim % 16 != 0 || num_tokens > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
  if (num_tokens == 0) return NIMBUS_OK;
  if (!qkv || !positions || !cos_table || !sin_table || !k_cache || !v_cache || !slot_mapping)
    return NIMBUS_ERR_INVALID;
  const int64_t row = (static_cast<int64_t>(num_heads) + 2 * num_kv_heads) * head_dim;
  if (qkv_stride < row || table_stride < head_dim) return NIMBUS_ERR_INVALID;
  if (qkv_stride % 8 != 0 || (reinterpret_cast<uintptr_t>(qkv) | reinterpret_cast<uintptr_t>(k_cache) |
                              reinterpret_cast<uintptr_t>(v_cache)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if (table_stride % 4 != 0 ||
      (reinterpret_cast<uintptr_t>(cos_table) | reinterpret_cast<uintptr_t>(sin_table)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  RopeWriteArgs w;
  w.r.x = static_cast<uint16_t*>(qkv);
  w.r.sx = qkv_stride;
  w.r.pos = positions;
  w.r.cos = cos_table;
  w.r.sin = sin_table;
  w.r.st = table_stride;
  w.r.tokens = static_cast<int32_t>(num_tokens);
  w.r.heads = num_heads + num_kv_heads;
  w.r.d = head_dim;
  w.r.max_pos = max_position;
  w.q_heads = num_heads;
  w.kv_heads = num_kv_heads;
  w.kc = static_cast<uint16_t*>(k_cache);
  w.vc = static_cast<uint16_t*>(v_cache);
  w.slots = slot_mapping;
  w.num_slots = num_slots;
  const int64_t threads = num_tokens * w.r.heads * (head_dim / 16);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kFloat16) {
    hipLaunchKernelGGL((rope_write_kv_kernel<kFloat16>), grid, dim3(256), 0, s, w);
  } else {
    hipLaunchKernelGGL((rope_write_kv_kernel<kBFloat16>), grid, dim3(256), 0, s, w);
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int nimbus_silu_mul(const void* x, int64_t x_stride, void* out, int64_t out_stride, int64_t rows,
                               int32_t cols, int32_t dtype, void* stream) {
  if (rows < 0 || cols <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (cols % 8 != 0 || rows > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
  if (rows == 0) return NIMBUS_OK;
  if (!x || !out) return NIMBUS_ERR_INVALID;
  if (x_stride < 2 * static_cast<int64_t>(cols) || out_stride < cols) return NIMBUS_ERR_INVALID;
  if ((x_stride | out_stride) % 8 != 0 ||
      (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  SiluArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.sx = x_stride;
  a.out = static_cast<uint16_t*>(out);
  a.so = out_stride;
  a.rows = static_cast<int32_t>(rows);
  a.cols = cols;
  const int64_t threads = rows * (cols / 8);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kFloat16) {
    hipLaunchKernelGGL((silu_mul_kernel<kFloat16>), grid, dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((silu_mul_kernel<kBFloat16>), grid, dim3(256), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}
