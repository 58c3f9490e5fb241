// Paged decode attention for gfx950: one query token per sequence, GQA.
//
// Replaces nimbus/kernels/paged_attention.py:25-146 (the Triton
// _paged_decode_kernel, _merge_partitions_kernel and their wrapper).
//
// Work split. The context of every sequence is cut into partitions of
// PART tokens (page aligned). One workgroup of four waves owns one
// (partition, kv head, sequence) and serves every query head that shares the
// kv head, so each K/V page is read from HBM exactly once. Inside the
// workgroup, wave w takes the 32-token chunks (two 16-token pages) w, w+4, ...
// The launch grid is (ceil(max_context / PART), KV * ceil(G / 16), B): it depends
// only on host integers, so a call is capturable in a hipGraph; partitions
// past a sequence's end exit at once.
//
// Per chunk, with G query heads padded to 16 MFMA columns:
//   S^T[token][g] = K[token][:] . Q^T[:][g]   (16x16x32 MFMA, K straight from
//                                               HBM into the A-operand layout)
//   online softmax per column g in fp32 (exp2 domain), reductions across the
//   four 16-lane groups with lane shuffles
//   O^T[d][g]    += V^T[d][token] . P^T[token][g]  (16x16x16 fp16 MFMA; P^T
//                                               is the QK output layout as is;
//                                               V is converted to fp16 while
//                                               staged through LDS, read
//                                               transposed)
// The four waves' partial (m, l, O) are merged through LDS. A sequence that
// fits in one partition is normalised and written directly; otherwise the
// partition writes fp32 (O, m, l) and paged_decode_merge_kernel combines
// them (empty partitions never exist: a partition index below
// ceil(ctx / PART) always holds at least one token).
#include "common.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

constexpr int kDecodeWaves = 4;
constexpr int kDecodeThreads = 64 * kDecodeWaves;
constexpr int kChunk = 32;  // tokens per wave iteration: two pages

struct DecodeArgs {
  const uint16_t* q;
  int64_t q_sb, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t c_sb, c_st, c_sh;
  const int32_t* bt;
  int64_t bt_sb;
  int32_t bt_width;
  int32_t num_blocks;
  const int32_t* ctx;
  uint16_t* out;
  int64_t o_sb, o_sh;
  float* part_o;   // [B, H, P, D]
  float* part_ml;  // [B, H, P, 2]
  int32_t H, G, gchunks, P;
  float scale_log2;
};

// LDS: per-wave staging of one chunk of V, later reused for the cross-wave merge.
template <int D>
struct DecodeSmem {
  static constexpr int kVRow = D + 4;  // u16 stride; rows 4 apart land on different banks
  static constexpr int kVBytes = kDecodeWaves * kChunk * kVRow * 2;
  static constexpr int kMergeBytes = kDecodeWaves * (16 * D + 32) * 4;
  static constexpr int kBytes = kVBytes > kMergeBytes ? kVBytes : kMergeBytes;
};

__device__ __forceinline__ int clamp_page(int32_t pid, int32_t nb) {
  return static_cast<uint32_t>(pid) < static_cast<uint32_t>(nb) ? pid : 0;
}

template <int DT, int D, int PART>
__global__ __launch_bounds__(kDecodeThreads) void paged_decode_kernel(DecodeArgs a) {
  constexpr int KK = D / 32;              // 16x16x32 steps over the head dim
  constexpr int NN = D / 16;              // 16-row blocks of O^T
  constexpr int LPT = D / 8;              // lanes per token row (16 bytes each)
  constexpr int TPL = 64 / LPT;           // token rows per wave-wide load
  constexpr int VLOADS = kChunk / TPL;    // 16-byte V loads per lane per chunk
  constexpr int VROW = DecodeSmem<D>::kVRow;
  __shared__ __attribute__((aligned(16))) unsigned char smem[DecodeSmem<D>::kBytes];

  const int part = blockIdx.x;
  const int kvh = blockIdx.y / a.gchunks;
  const int g0 = (blockIdx.y % a.gchunks) * 16;
  const int b = blockIdx.z;

  int ctx = a.ctx[b];
  ctx = min(ctx, min(a.P * PART, a.bt_width * 16));
  const int n_parts = (ctx + PART - 1) / PART;
  if (part >= n_parts) return;

  const int tok0 = part * PART;
  const int tok1 = min(tok0 + PART, ctx);
  const int n_pages = (tok1 - tok0 + 15) / 16;
  const int n_chunks = (n_pages + 1) / 2;

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int col = lane % 16;
  const int grp = lane / 16;
  const int g = g0 + col;
  const bool g_ok = g < a.G;
  const int h = kvh * a.G + (g_ok ? g : 0);

  // Q^T as the B operand: column g, k-group grp holds q[g][32kk + 8grp .. +8].
  u32x4 qop[KK];
  {
    const uint16_t* qrow = a.q + b * a.q_sb + static_cast<int64_t>(h) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      u32x4 v = *reinterpret_cast<const u32x4*>(qrow + 32 * kk + 8 * grp);
      qop[kk] = g_ok ? v : u32x4{0, 0, 0, 0};
    }
  }

  const int32_t* btrow = a.bt + b * a.bt_sb + tok0 / 16;
  const uint16_t* kbase = a.kc + static_cast<int64_t>(kvh) * a.c_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(kvh) * a.c_sh;
  uint16_t* vb = reinterpret_cast<uint16_t*>(smem) + wave * kChunk * VROW;

  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4 acc[NN];
#pragma unroll
  for (int nn = 0; nn < NN; ++nn) acc[nn] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Registers of one chunk: K in A-operand layout, V rows as loaded.
  u32x4 kreg[2][KK];
  u32x4 vreg[VLOADS];

  auto load_chunk = [&](int c) {
    const int p0 = 2 * c;
    const bool has1 = p0 + 1 < n_pages;
    const int pid0 = clamp_page(btrow[p0], a.num_blocks);
    const int pid1 = has1 ? clamp_page(btrow[p0 + 1], a.num_blocks) : pid0;
    const int64_t off0 = static_cast<int64_t>(pid0) * a.c_sb;
    const int64_t off1 = static_cast<int64_t>(pid1) * a.c_sb;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      kreg[0][kk] = *reinterpret_cast<const u32x4*>(kbase + off0 + col * a.c_st + 32 * kk + 8 * grp);
    }
    if (has1) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        kreg[1][kk] = *reinterpret_cast<const u32x4*>(kbase + off1 + col * a.c_st + 32 * kk + 8 * grp);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) kreg[1][kk] = u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int tt = r * TPL + lane / LPT;
      const int cc = lane % LPT;
      const bool second = tt >= 16;
      if (!second || has1) {
        const int64_t off = second ? off1 : off0;
        vreg[r] = *reinterpret_cast<const u32x4*>(vbase + off + (tt % 16) * a.c_st + 8 * cc);
      } else {
        vreg[r] = u32x4{0, 0, 0, 0};
      }
    }
  };

  int c = wave;
  if (c < n_chunks) load_chunk(c);
  for (; c < n_chunks; c += kDecodeWaves) {
    // Stage V (zeroing rows past the context: 0 * garbage must not reach the sum).
    const int valid = tok1 - (tok0 + kChunk * c);
#pragma unroll
    for (int r = 0; r < VLOADS; ++r) {
      const int tt = r * TPL + lane / LPT;
      const int cc = lane % LPT;
      u32x4 v = tt < valid ? vreg[r] : u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = v_to_f16_pair<DT>(v[e]);
      u32x2* dst = reinterpret_cast<u32x2*>(vb + tt * VROW + 8 * cc);
      dst[0] = u32x2{v[0], v[1]};
      dst[1] = u32x2{v[2], v[3]};
    }
    // S^T for both pages.
    f32x4 s[2];
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) t = mfma_16x16x32<DT>(kreg[pi][kk], qop[kk], t);
      s[pi] = t;
    }
    // Next chunk's loads go out before the softmax and PV of this one.
    if (c + kDecodeWaves < n_chunks) load_chunk(c + kDecodeWaves);

    float mx = -INFINITY;
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * pi + 4 * grp + r;
        const float x = t < valid ? s[pi][r] * a.scale_log2 : -INFINITY;
        s[pi][r] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = max_across_groups(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = exp2f(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
    u32x2 pop[2];
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = exp2f(s[pi][r] - m_new);
        psum += p[r];
      }
      pop[pi] = u32x2{pack2(f32_to_f16(p[0]), f32_to_f16(p[1])), pack2(f32_to_f16(p[2]), f32_to_f16(p[3]))};
    }
    l_run = l_run * alpha + psum;
#pragma unroll
    for (int nn = 0; nn < NN; ++nn) acc[nn] *= alpha;

    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      const uint16_t* vrow = vb + (16 * pi + 4 * grp) * VROW + col;
#pragma unroll
      for (int nn = 0; nn < NN; ++nn) {
        const uint16_t* p = vrow + 16 * nn;
        u32x2 vop = u32x2{pack2(p[0], p[VROW]), pack2(p[2 * VROW], p[3 * VROW])};
        acc[nn] = mfma_16x16x16<kFloat16>(vop, pop[pi], acc[nn]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  l_run = sum_across_groups(l_run);

  // Cross-wave merge through LDS (reusing the V staging space).
  __syncthreads();
  float* mo = reinterpret_cast<float*>(smem);          // [wave][16][D]
  float* mm = mo + kDecodeWaves * 16 * D;               // [wave][16]
  float* ml = mm + kDecodeWaves * 16;                   // [wave][16]
#pragma unroll
  for (int nn = 0; nn < NN; ++nn) {
#pragma unroll
    for (int r = 0; r < 4; ++r) mo[(wave * 16 + col) * D + 16 * nn + 4 * grp + r] = acc[nn][r];
  }
  if (grp == 0) {
    mm[wave * 16 + col] = m_run;
    ml[wave * 16 + col] = l_run;
  }
  __syncthreads();

  const int gcount = min(16, a.G - g0);
  const bool single = n_parts == 1;
  for (int idx = tid; idx < gcount * D; idx += kDecodeThreads) {
    const int cg = idx / D;
    const int d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) M = fmaxf(M, mm[w * 16 + cg]);
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kDecodeWaves; ++w) {
      const float wt = exp2f(mm[w * 16 + cg] - M);
      L += ml[w * 16 + cg] * wt;
      O += mo[(w * 16 + cg) * D + d] * wt;
    }
    const int hh = kvh * a.G + g0 + cg;
    if (single) {
      a.out[b * a.o_sb + static_cast<int64_t>(hh) * a.o_sh + d] = Elem<DT>::from_f32(O / L);
    } else {
      const int64_t row = (static_cast<int64_t>(b) * a.H + hh) * a.P + part;
      a.part_o[row * D + d] = O;
      if (d == 0) {
        a.part_ml[row * 2] = M;
        a.part_ml[row * 2 + 1] = L;
      }
    }
  }
}

// Second pass: combine a sequence's partitions, o = sum_p O_p w_p / sum_p L_p w_p
// with w_p = 2^(m_p - max m). One wave per (head, sequence).
template <int DT, int D, int PART>
__global__ __launch_bounds__(64) void paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int DPL = D / 64;
  const int hh = blockIdx.x;
  const int b = blockIdx.y;
  int ctx = a.ctx[b];
  ctx = min(ctx, min(a.P * PART, a.bt_width * 16));
  const int n = (ctx + PART - 1) / PART;
  if (n <= 1) return;
  const int64_t row0 = (static_cast<int64_t>(b) * a.H + hh) * a.P;
  float M = -INFINITY;
  for (int p = 0; p < n; ++p) M = fmaxf(M, a.part_ml[(row0 + p) * 2]);
  float L = 0.f;
  float O[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) O[i] = 0.f;
  const int lane = threadIdx.x;
  for (int p = 0; p < n; ++p) {
    const float wt = exp2f(a.part_ml[(row0 + p) * 2] - M);
    L += a.part_ml[(row0 + p) * 2 + 1] * wt;
#pragma unroll
    for (int i = 0; i < DPL; ++i) O[i] += a.part_o[(row0 + p) * D + lane * DPL + i] * wt;
  }
  const float inv = 1.f / L;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    a.out[b * a.o_sb + static_cast<int64_t>(hh) * a.o_sh + lane * DPL + i] = Elem<DT>::from_f32(O[i] * inv);
  }
}

// phase bit 1: partition pass, bit 2: merge pass.
template <int DT, int D, int PART>
static int launch_decode(const DecodeArgs& a, int batch, int kv_heads, int phases, hipStream_t stream) {
  if (phases & 1) {
    dim3 grid(a.P, kv_heads * a.gchunks, batch);
    hipLaunchKernelGGL((paged_decode_kernel<DT, D, PART>), grid, dim3(kDecodeThreads), 0, stream, a);
  }
  if ((phases & 2) && a.P > 1) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<DT, D, PART>), dim3(a.H, batch), dim3(64), 0, stream, a);
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace nimbus

using namespace nimbus;

extern "C" int64_t nimbus_paged_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim,
                                                       int64_t max_context) {
  if (batch < 0 || num_heads <= 0 || head_dim <= 0 || max_context < 0) return -1;
  const int64_t parts = (max_context + kDecodePartition - 1) / kDecodePartition;
  if (parts <= 1) return 0;
  return static_cast<int64_t>(batch) * num_heads * parts * (head_dim + 2) * 4;
}

static int paged_decode_impl(int phases, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                                   const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                   int64_t cache_stride_token, int64_t cache_stride_head,
                                   const int32_t* block_tables, int64_t bt_stride, int32_t bt_width,
                                   const int32_t* context_lens, void* out, int64_t out_stride_b,
                                   int64_t out_stride_h, void* workspace, int64_t workspace_bytes, int32_t batch,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                   int64_t max_context, float scale, int32_t dtype, void* stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return NIMBUS_ERR_INVALID;
  if (block_size != 16) return NIMBUS_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return NIMBUS_ERR_UNSUPPORTED;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (batch == 0 || max_context <= 0) return NIMBUS_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out) return NIMBUS_ERR_INVALID;
  if (num_blocks <= 0 || num_blocks > INT32_MAX || bt_width <= 0) return NIMBUS_ERR_INVALID;
  // 16-byte vector access: 8-element aligned strides and bases.
  if ((q_stride_b | q_stride_h | cache_stride_block | cache_stride_token | cache_stride_head) % 8 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
       reinterpret_cast<uintptr_t>(v_cache)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  const int64_t need = nimbus_paged_decode_workspace_bytes(batch, num_heads, head_dim, max_context);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return NIMBUS_ERR_WORKSPACE;
  const int64_t parts = (max_context + kDecodePartition - 1) / kDecodePartition;
  if (parts > INT32_MAX / 16 || batch > 65535) return NIMBUS_ERR_UNSUPPORTED;

  DecodeArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.c_sb = cache_stride_block;
  a.c_st = cache_stride_token;
  a.c_sh = cache_stride_head;
  a.bt = block_tables;
  a.bt_sb = bt_stride;
  a.bt_width = bt_width;
  a.num_blocks = static_cast<int32_t>(num_blocks);
  a.ctx = context_lens;
  a.out = static_cast<uint16_t*>(out);
  a.o_sb = out_stride_b;
  a.o_sh = out_stride_h;
  a.part_o = static_cast<float*>(workspace);
  a.part_ml = need > 0 ? a.part_o + static_cast<int64_t>(batch) * num_heads * parts * head_dim : nullptr;
  a.H = num_heads;
  a.G = num_heads / num_kv_heads;
  a.gchunks = (a.G + 15) / 16;
  a.P = static_cast<int32_t>(parts);
  a.scale_log2 = scale * 1.4426950408889634f;
  if (num_kv_heads * a.gchunks > 65535) return NIMBUS_ERR_UNSUPPORTED;

  hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr int P = kDecodePartition;
  if (dtype == kFloat16) {
    return head_dim == 64 ? launch_decode<kFloat16, 64, P>(a, batch, num_kv_heads, phases, s)
                          : launch_decode<kFloat16, 128, P>(a, batch, num_kv_heads, phases, s);
  }
  return head_dim == 64 ? launch_decode<kBFloat16, 64, P>(a, batch, num_kv_heads, phases, s)
                        : launch_decode<kBFloat16, 128, P>(a, batch, num_kv_heads, phases, s);
}

#define NIMBUS_DECODE_PARAMS                                                                                    \
  const void *q, int64_t q_stride_b, int64_t q_stride_h, const void *k_cache, const void *v_cache,              \
      int64_t num_blocks, int64_t cache_stride_block, int64_t cache_stride_token, int64_t cache_stride_head,    \
      const int32_t *block_tables, int64_t bt_stride, int32_t bt_width, const int32_t *context_lens, void *out, \
      int64_t out_stride_b, int64_t out_stride_h, void *workspace, int64_t workspace_bytes, int32_t batch,      \
      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, int64_t max_context,      \
      float scale, int32_t dtype, void *stream
#define NIMBUS_DECODE_ARGS                                                                                  \
  q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks, cache_stride_block, cache_stride_token,          \
      cache_stride_head, block_tables, bt_stride, bt_width, context_lens, out, out_stride_b, out_stride_h,   \
      workspace, workspace_bytes, batch, num_heads, num_kv_heads, head_dim, block_size, max_context, scale, \
      dtype, stream

extern "C" int nimbus_paged_decode(NIMBUS_DECODE_PARAMS) { return paged_decode_impl(3, NIMBUS_DECODE_ARGS); }

extern "C" int nimbus_paged_decode_partitions(NIMBUS_DECODE_PARAMS) {
  return paged_decode_impl(1, NIMBUS_DECODE_ARGS);
}

extern "C" int nimbus_paged_decode_merge(NIMBUS_DECODE_PARAMS) { return paged_decode_impl(2, NIMBUS_DECODE_ARGS); }
