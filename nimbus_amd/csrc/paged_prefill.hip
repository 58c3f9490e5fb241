// Causal varlen paged prefill attention for gfx950.
//
// Replaces nimbus/kernels/prefill_attention.py:25-119 (the Triton
// _paged_prefill_kernel and its wrapper).
//
// Query j of sequence i (q_len = query_start[i+1] - query_start[i],
// ctx = context_lens[i]) sits at absolute position ctx - q_len + j and
// attends to cached keys 0..ctx - q_len + j, read through the block table.
//
// Work split. One workgroup owns one tile-table entry (sequence, 64 query
// positions starting at m0), one kv head and GS of the G query heads that
// share it: 64 * GS rows, 32 per wave, row r = position r / GS, head r % GS.
// Stacking the GQA heads as rows means every K/V tile is read from HBM once
// per GS heads instead of once per head (the Triton grid is (tiles, H)).
//
// Per 64-key block: the workgroup stages K (row-major) and V (transposed,
// V^T[d][key]) in LDS, then each wave computes
//   S^T[key][row] = K[key][:] . Q^T[:][row]    16x16x32 MFMA, Q^T in registers
//   online softmax per row in fp32 (exp2 domain)
//   O^T[d][row]  += V^T[d][key] . P^T[key][row] 16x16x32 fp16 MFMA; P^T is
//                                               the QK output layout as is,
//                                               V^T is converted to fp16 when
//                                               staged
// Waves skip key blocks that lie entirely after their last query position.
#include "common.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

constexpr int kBlockN = 64;  // keys per iteration (four pages)

struct PrefillArgs {
  const uint16_t* q;
  int64_t q_st, q_sh;
  const uint16_t* kc;
  const uint16_t* vc;
  int64_t c_sb, c_st, c_sh;
  const int32_t* bt;
  int64_t bt_sb;
  int32_t bt_width;
  int32_t num_blocks;
  const int32_t* qstart;
  const int32_t* ctx;
  const int32_t* prog_seq;
  const int32_t* prog_m;
  uint16_t* out;
  int64_t o_st, o_sh;
  int32_t G, gsplit;
  float scale_log2;
};

template <int D>
struct PrefillSmem {
  static constexpr int kKRow = D + 8;        // u16 stride of K rows (16-byte aligned, rows rotate banks)
  static constexpr int kVRow = kBlockN + 4;  // u16 stride of V^T rows
  static constexpr int kBytes = (kBlockN * kKRow + D * kVRow) * 2;
};

template <int DT, int D, int GS>
__global__ __launch_bounds__(128 * GS) void paged_prefill_kernel(PrefillArgs a) {
  constexpr int NT = 128 * GS;              // threads
  constexpr int KK = D / 32;                // 16x16x32 steps over the head dim (QK)
  constexpr int ND = D / 16;                // 16-row blocks of O^T
  constexpr int PIECES = kBlockN * D / 8;   // 16-byte pieces in one K (or V) tile
  constexpr int PPT = PIECES / NT;          // pieces per thread
  constexpr int KROW = PrefillSmem<D>::kKRow;
  constexpr int VROW = PrefillSmem<D>::kVRow;
  static_assert(PIECES % NT == 0, "tile pieces must divide evenly");
  __shared__ __attribute__((aligned(16))) uint16_t smem[PrefillSmem<D>::kBytes / 2];
  uint16_t* ks = smem;                      // [kBlockN][KROW]
  uint16_t* vts = smem + kBlockN * KROW;    // [D][VROW]

  const int prog = blockIdx.x;
  const int kvh = blockIdx.y / a.gsplit;
  const int gsub = blockIdx.y % a.gsplit;
  const int seq = a.prog_seq[prog];
  const int m0 = a.prog_m[prog];
  const int qs = a.qstart[seq];
  const int q_len = a.qstart[seq + 1] - qs;
  int ctx = a.ctx[seq];
  ctx = min(ctx, a.bt_width * 16);
  const int base_pos = ctx - q_len;  // absolute position of query 0
  const int kv_end = max(0, min(ctx, base_pos + m0 + 64));

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int col = lane % 16;
  const int grp = lane / 16;

  // This lane's two rows (one per 16-row N block).
  int qpos[2];
  bool row_ok[2];
  int head[2];
  int64_t qoff[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int r = 32 * wave + 16 * nb + col;
    const int pos = r / GS;
    const int gi = r % GS;
    row_ok[nb] = m0 + pos < q_len;
    qpos[nb] = base_pos + m0 + pos;
    head[nb] = kvh * a.G + gsub * GS + gi;
    qoff[nb] = static_cast<int64_t>(qs + m0 + pos) * a.q_st + static_cast<int64_t>(head[nb]) * a.q_sh;
  }
  const int wave_last_pos = min(32 * (wave + 1) / GS, 64) - 1;
  const int wave_kv_end = min(kv_end, base_pos + m0 + wave_last_pos + 1);

  // Q^T as the B operand.
  u32x4 qop[2][KK];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      qop[nb][kk] = row_ok[nb] ? *reinterpret_cast<const u32x4*>(a.q + qoff[nb] + 32 * kk + 8 * grp)
                               : u32x4{0, 0, 0, 0};
    }
  }

  const int32_t* btrow = a.bt + seq * a.bt_sb;
  const uint16_t* kbase = a.kc + static_cast<int64_t>(kvh) * a.c_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(kvh) * a.c_sh;

  float m_run[2] = {-INFINITY, -INFINITY};
  float l_run[2] = {0.f, 0.f};
  f32x4 acc[ND][2];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) {
    acc[nd][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[nd][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  u32x4 kreg[PPT], vreg[PPT];
  auto load_tile = [&](int kb) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + NT * i;
      const int key = p / (D / 8);
      const int dc = p % (D / 8);
      const int t = kb * kBlockN + key;
      if (t < kv_end) {
        int pid = btrow[t / 16];
        pid = static_cast<uint32_t>(pid) < static_cast<uint32_t>(a.num_blocks) ? pid : 0;
        const int64_t off = static_cast<int64_t>(pid) * a.c_sb + (t % 16) * a.c_st + 8 * dc;
        kreg[i] = *reinterpret_cast<const u32x4*>(kbase + off);
        vreg[i] = *reinterpret_cast<const u32x4*>(vbase + off);
      } else {
        kreg[i] = u32x4{0, 0, 0, 0};
        vreg[i] = u32x4{0, 0, 0, 0};
      }
    }
  };

  const int n_kb = (kv_end + kBlockN - 1) / kBlockN;
  if (n_kb > 0) load_tile(0);
  for (int kb = 0; kb < n_kb; ++kb) {
    __syncthreads();  // every wave is done reading the previous tile
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + NT * i;
      const int key = p / (D / 8);
      const int dc = p % (D / 8);
      *reinterpret_cast<u32x4*>(ks + key * KROW + 8 * dc) = kreg[i];
      u32x4 v = vreg[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = v_to_f16_pair<DT>(v[e]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vts[(8 * dc + 2 * e) * VROW + key] = static_cast<uint16_t>(v[e] & 0xffffu);
        vts[(8 * dc + 2 * e + 1) * VROW + key] = static_cast<uint16_t>(v[e] >> 16);
      }
    }
    __syncthreads();
    if (kb + 1 < n_kb) load_tile(kb + 1);

    const int key0 = kb * kBlockN;
    if (key0 >= wave_kv_end) continue;  // every key of this block is after this wave's queries

    // S^T[key][row], four 16-key blocks x two 16-row blocks.
    f32x4 s[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      s[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const u32x4 kop = *reinterpret_cast<const u32x4*>(ks + (16 * mb + col) * KROW + 32 * kk + 8 * grp);
        s[mb][0] = mfma_16x16x32<DT>(kop, qop[0][kk], s[mb][0]);
        s[mb][1] = mfma_16x16x32<DT>(kop, qop[1][kk], s[mb][1]);
      }
    }

    u32x4 pop[2][2];  // [key chunk of 32][row block]
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float mx = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = key0 + 16 * mb + 4 * grp + r;
          const bool ok = t <= qpos[nb] && t < kv_end;
          const float x = ok ? s[mb][nb][r] * a.scale_log2 : -INFINITY;
          s[mb][nb][r] = x;
          mx = fmaxf(mx, x);
        }
      }
      mx = max_across_groups(mx);
      const float m_new = fmaxf(m_run[nb], mx);
      const float m_safe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m_run[nb] - m_safe);
      m_run[nb] = m_new;
      float psum = 0.f;
      uint16_t ph[4][4];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = exp2f(s[mb][nb][r] - m_safe);
          psum += p;
          ph[mb][r] = f32_to_f16(p);
        }
      }
      l_run[nb] = l_run[nb] * alpha + psum;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) acc[nd][nb] *= alpha;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        pop[kc][nb] = u32x4{pack2(ph[2 * kc][0], ph[2 * kc][1]), pack2(ph[2 * kc][2], ph[2 * kc][3]),
                            pack2(ph[2 * kc + 1][0], ph[2 * kc + 1][1]), pack2(ph[2 * kc + 1][2], ph[2 * kc + 1][3])};
      }
    }

    // O^T[d][row] += V^T[d][key] P^T[key][row]
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      const uint16_t* vrow = vts + (16 * nd + col) * VROW;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow + 32 * kc + 4 * grp);
        const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 32 * kc + 16 + 4 * grp);
        const u32x4 vop = u32x4{lo[0], lo[1], hi[0], hi[1]};
        acc[nd][0] = mfma_16x16x32<kFloat16>(vop, pop[kc][0], acc[nd][0]);
        acc[nd][1] = mfma_16x16x32<kFloat16>(vop, pop[kc][1], acc[nd][1]);
      }
    }
  }

#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float l = sum_across_groups(l_run[nb]);
    if (!row_ok[nb]) continue;
    const float inv = l == 0.f ? 0.f : 1.f / l;
    uint16_t* orow = a.out + static_cast<int64_t>(qs + m0 + (32 * wave + 16 * nb + col) / GS) * a.o_st +
                     static_cast<int64_t>(head[nb]) * a.o_sh;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
      const f32x4 o = acc[nd][nb];
      const u32x2 w = u32x2{pack2(Elem<DT>::from_f32(o[0] * inv), Elem<DT>::from_f32(o[1] * inv)),
                            pack2(Elem<DT>::from_f32(o[2] * inv), Elem<DT>::from_f32(o[3] * inv))};
      *reinterpret_cast<u32x2*>(orow + 16 * nd + 4 * grp) = w;
    }
  }
}

template <int DT, int D, int GS>
static int launch_prefill(const PrefillArgs& a, int num_programs, int kv_heads, hipStream_t stream) {
  dim3 grid(num_programs, kv_heads * a.gsplit);
  hipLaunchKernelGGL((paged_prefill_kernel<DT, D, GS>), grid, dim3(128 * GS), 0, stream, a);
  return static_cast<int>(hipGetLastError());
}

template <int DT, int D>
static int dispatch_gs(const PrefillArgs& a, int gs, int num_programs, int kv_heads, hipStream_t s) {
  switch (gs) {
    case 1:
      return launch_prefill<DT, D, 1>(a, num_programs, kv_heads, s);
    case 2:
      return launch_prefill<DT, D, 2>(a, num_programs, kv_heads, s);
    default:
      return launch_prefill<DT, D, 4>(a, num_programs, kv_heads, s);
  }
}

}  // namespace nimbus

using namespace nimbus;

extern "C" int nimbus_paged_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                    const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                    int64_t cache_stride_token, int64_t cache_stride_head,
                                    const int32_t* block_tables, int64_t bt_stride, int32_t bt_width,
                                    const int32_t* query_start, const int32_t* context_lens,
                                    const int32_t* prog_seq, const int32_t* prog_m, int32_t num_programs,
                                    void* out, int64_t out_stride_t, int64_t out_stride_h, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                    int32_t dtype, void* stream) {
  if (num_programs < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return NIMBUS_ERR_INVALID;
  if (block_size != 16) return NIMBUS_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return NIMBUS_ERR_UNSUPPORTED;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  const int G = num_heads / num_kv_heads;
  const int gs = G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1);
  if (num_programs == 0) return NIMBUS_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !query_start || !context_lens || !prog_seq || !prog_m || !out)
    return NIMBUS_ERR_INVALID;
  if (num_blocks <= 0 || num_blocks > INT32_MAX || bt_width <= 0) return NIMBUS_ERR_INVALID;
  if ((q_stride_t | q_stride_h | cache_stride_block | cache_stride_token | cache_stride_head | out_stride_t |
       out_stride_h) % 8 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
       reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if (num_kv_heads * (G / gs) > 65535) return NIMBUS_ERR_UNSUPPORTED;

  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q);
  a.q_st = q_stride_t;
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
  a.qstart = query_start;
  a.ctx = context_lens;
  a.prog_seq = prog_seq;
  a.prog_m = prog_m;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.G = G;
  a.gsplit = G / gs;
  a.scale_log2 = scale * 1.4426950408889634f;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kFloat16) {
    return head_dim == 64 ? dispatch_gs<kFloat16, 64>(a, gs, num_programs, num_kv_heads, s)
                          : dispatch_gs<kFloat16, 128>(a, gs, num_programs, num_kv_heads, s);
  }
  return head_dim == 64 ? dispatch_gs<kBFloat16, 64>(a, gs, num_programs, num_kv_heads, s)
                        : dispatch_gs<kBFloat16, 128>(a, gs, num_programs, num_kv_heads, s);
}
