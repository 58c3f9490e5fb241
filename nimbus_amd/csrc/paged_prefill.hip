// Causal varlen paged prefill attention for gfx950.
//
// Replaces nimbus/kernels/prefill_attention.py:25-119 (the Triton
// _paged_prefill_kernel and its wrapper).
//
// Query j of sequence i (q_len = query_start[i+1] - query_start[i],
// ctx = context_lens[i]) sits at absolute position ctx - q_len + j and
// attends to cached keys 0..ctx - q_len + j, read through the block table.
//
// Work units. A tile-table entry (sequence, 64 query positions from m0,
// the reference's BLOCK_M) is cut into units of POS positions; a unit covers
// one kv head and GS of the G query heads that share it, stacked as rows:
// POS * GS = 128 rows (64 when GS = 1), 32 per wave, row r = position
// r / GS, head r % GS. Stacking the GQA heads means every K/V tile is read
// once per GS heads instead of once per head (the Triton grid is (tiles, H)).
// The kv-head group varies fastest over the grid, so consecutive
// workgroups, which the dispatcher spreads over the eight XCDs, keep one kv
// head per XCD and its K/V in that XCD's L2; the host orders the tile table
// by cost (heavy entries first, the light half reversed) so that the two
// workgroups sharing a CU tend to carry a heavy and a light unit.
//
// Per 64-key block the workgroup stages K and V (fp16; bf16 V converted)
// into LDS, double-buffered, with XOR-swizzled 16-byte chunks; the next
// block's global loads are in flight while the current one is computed.
// Each wave then computes, for its 32 rows:
//   S^T[key][row] = K[key][:] . Q^T[:][row]   16x16x32 MFMA, K read from LDS
//                                              in the A-operand layout, Q^T in
//                                              registers
//   softmax in the exp2 domain with a lazily raised running max: the max
//   only moves when a score exceeds it by more than 2^8, so the rescale of
//   O is rare and P = 2^(s - m) stays below 256 (exact range in fp16); row
//   sums stay per lane until the end
//   O^T[d][row]  += V^T[d][key] . P^T[key][row]  16x16x32 fp16 MFMA, V^T read
//                                              with ds_read_b64_tr_b16, P^T is
//                                              the QK output layout as is
// Causal and context masks are applied only on blocks that need them.
#include "common.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

constexpr int kBlockN = 64;        // keys per iteration (four pages)
constexpr float kLazyMax = 8.f;    // log2 headroom before the running max moves

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
  int32_t G, gsplit, kvg;
  float scale_log2;
};

template <int GS>
struct PrefillShape {
  static constexpr int kPos = 128 / GS < kPrefillTile ? 128 / GS : kPrefillTile;  // positions per unit
  static constexpr int kRows = kPos * GS;
  static constexpr int kWaves = kRows / 32;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kSub = kPrefillTile / kPos;  // units per tile-table entry
};

// Swizzled 16-byte chunk positions of the LDS tiles. K rows are read sixteen
// at a time (one key per lane column) by the QK operand loads; V rows sixteen
// at a time by the transposed reads. XOR-ing the chunk index with a function
// of the row spreads equal chunks of those rows over the LDS banks.
template <int D>
__device__ __forceinline__ int k_pos(int key, int c) {
  return c ^ (key & (D / 8 - 1));
}
template <int D>
__device__ __forceinline__ int v_pos(int key, int c) {
  return c ^ ((2 * key) & (D / 8 - 1));
}

__device__ __forceinline__ int32_t scalar_load_i32(const int32_t* p, int i) {
  typedef const __attribute__((address_space(4))) int32_t* const_ptr;
  return ((const_ptr)(p))[i];
}

template <int DT, int D, int GS>
__global__ __launch_bounds__(PrefillShape<GS>::kThreads) __attribute__((amdgpu_waves_per_eu(2))) void
paged_prefill_kernel(PrefillArgs a) {
  using Shape = PrefillShape<GS>;
  constexpr int NT = Shape::kThreads;
  constexpr int POS = Shape::kPos;
  constexpr int KK = D / 32;                // 16x16x32 steps over the head dim (QK)
  constexpr int ND = D / 16;                // 16-row blocks of O^T
  constexpr int CPR = D / 8;                // 16-byte chunks per K/V row
  constexpr int PIECES = kBlockN * CPR;     // 16-byte pieces in one K (or V) tile
  constexpr int PPT = PIECES / NT;          // pieces per thread
  constexpr int TILE = kBlockN * D;         // u16 elements of one tile
  static_assert(PIECES % NT == 0, "tile pieces must divide evenly");
  __shared__ __attribute__((aligned(16))) uint16_t ks[2 * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t vs[2 * TILE];

  // Unit: kv-head group fastest, then the sub-tile, then the table entry.
  const int kvg_id = blockIdx.x % a.kvg;
  const int r_unit = blockIdx.x / a.kvg;
  const int entry = r_unit / Shape::kSub;
  const int sub = r_unit % Shape::kSub;
  const int kvh = kvg_id / a.gsplit;
  const int gsub = kvg_id % a.gsplit;
  const int seq = a.prog_seq[entry];
  const int m0 = a.prog_m[entry] + sub * POS;
  const int qs = a.qstart[seq];
  const int q_len = a.qstart[seq + 1] - qs;
  if (m0 >= q_len) return;  // the whole workgroup: this sub-tile has no queries
  const int ctx = min(a.ctx[seq], a.bt_width * 16);
  const int base_pos = ctx - q_len;  // absolute position of query 0
  const int kv_end = max(0, min(ctx, base_pos + m0 + POS));
  const int n_kb = (kv_end + kBlockN - 1) / kBlockN;

  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int col = lane % 16;
  const int grp = lane / 16;

  // This lane's two rows (one per 16-row N block).
  int qpos[2], head[2];
  bool row_ok[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int r = 32 * wave + 16 * nb + col;
    const int pos = r / GS;
    row_ok[nb] = m0 + pos < q_len;
    qpos[nb] = base_pos + m0 + pos;
    head[nb] = kvh * a.G + gsub * GS + r % GS;
  }
  // Keys this wave's rows can see: [0, wave_end); blocks wholly below
  // wave_lo need no causal mask.
  const int wave_pos_lo = (32 * wave) / GS;
  const int wave_pos_hi = min((32 * wave + 31) / GS, q_len - 1 - m0);
  const int wave_end = wave_pos_lo > q_len - 1 - m0 ? 0 : min(kv_end, base_pos + m0 + wave_pos_hi + 1);
  const int wave_lo = base_pos + m0 + wave_pos_lo;

  // Q^T as the B operand (rows past q_len load the last query row).
  u32x4 qop[2][KK];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int pos = min((32 * wave + 16 * nb + col) / GS, q_len - 1 - m0);
    const uint16_t* qrow = a.q + static_cast<int64_t>(qs + m0 + pos) * a.q_st + static_cast<int64_t>(head[nb]) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qop[nb][kk] = *reinterpret_cast<const u32x4*>(qrow + 32 * kk + 8 * grp);
  }

  const int32_t* btrow = a.bt + seq * a.bt_sb;
  const uint16_t* kbase = a.kc + static_cast<int64_t>(kvh) * a.c_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(kvh) * a.c_sh;
  const int last_page = (kv_end + 15) / 16 - 1;

  // Staging registers of one block: piece p = tid + NT * i is key p / CPR,
  // chunk p % CPR.
  u32x4 kreg[PPT], vreg[PPT];
  auto load_block = [&](int kb) {
    const int k0 = kb * kBlockN;
    int pid[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int page = min(k0 / 16 + i, last_page);
      const int v = scalar_load_i32(btrow, page);
      pid[i] = static_cast<uint32_t>(v) < static_cast<uint32_t>(a.num_blocks) ? v : 0;
    }
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + NT * i;
      const int key = p / CPR;
      const int c = p % CPR;
      const int j = key / 16;
      const int page_id = j == 0 ? pid[0] : j == 1 ? pid[1] : j == 2 ? pid[2] : pid[3];
      const int64_t off = static_cast<int64_t>(page_id) * a.c_sb + (key % 16) * a.c_st + 8 * c;
      kreg[i] = *reinterpret_cast<const u32x4*>(kbase + off);
      vreg[i] = *reinterpret_cast<const u32x4*>(vbase + off);
    }
  };
  auto store_block = [&](int kb, int buf) {
    const int k0 = kb * kBlockN;
    const bool tail = k0 + kBlockN > kv_end;
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      const int p = tid + NT * i;
      const int key = p / CPR;
      const int c = p % CPR;
      u32x4 v = vreg[i];
      // Keys past the context: P is 0 there, but 0 * garbage must not reach the sum.
      if (tail && k0 + key >= kv_end) v = u32x4{0, 0, 0, 0};
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = v_to_f16_pair<DT>(v[e]);
      *reinterpret_cast<u32x4*>(ks + buf * TILE + key * D + 8 * k_pos<D>(key, c)) = kreg[i];
      *reinterpret_cast<u32x4*>(vs + buf * TILE + key * D + 8 * v_pos<D>(key, c)) = v;
    }
  };

  float m_run[2] = {-INFINITY, -INFINITY};
  float l_lane[2] = {0.f, 0.f};
  f32x4 acc[ND][2];
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) {
    acc[nd][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[nd][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Transposed-read addresses (see lds_read_tr16): lane j of group grp reads
  // V row 16 mb + 4 grp + j/4, elements 16 nd + 4 (j%4) .. +4.
  const int tr_row = 4 * grp + col / 4;
  const int tr_half = 4 * ((col % 4) % 2);
  const int tr_chunk = (col % 4) / 2;

  auto compute_block = [&](int kb, int buf) {
    const int k0 = kb * kBlockN;
    const uint16_t* kt = ks + buf * TILE;
    const uint16_t* vt = vs + buf * TILE;
    f32x4 s[4][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      s[mb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[mb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int key = 16 * mb + col;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const u32x4 kop = *reinterpret_cast<const u32x4*>(kt + key * D + 8 * k_pos<D>(key, 4 * kk + grp));
        s[mb][0] = mfma_16x16x32<DT>(kop, qop[0][kk], s[mb][0]);
        s[mb][1] = mfma_16x16x32<DT>(kop, qop[1][kk], s[mb][1]);
      }
    }
    // Mask (raw scores; only blocks that reach past a row's position or the
    // context need it), then lane-local maxima of the raw scores.
    const bool full = k0 + kBlockN - 1 <= wave_lo && k0 + kBlockN <= kv_end;
    if (!full) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int lim = min(qpos[nb] + 1, kv_end) - k0 - 4 * grp;  // key offsets below lim are visible
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
          for (int r = 0; r < 4; ++r) s[mb][nb][r] = 16 * mb + r < lim ? s[mb][nb][r] : -INFINITY;
        }
      }
    }
    float lm[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      float m = s[0][nb][0];
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) m = fmaxf(m, s[mb][nb][r]);
      }
      lm[nb] = m * a.scale_log2;  // the scale is positive: max commutes with it
    }
    // Lazy running max (exp2 domain): move it, and rescale O and the sums,
    // only when a score is more than 2^kLazyMax above it; P <= 2^kLazyMax.
    if (__builtin_amdgcn_ballot_w64(lm[0] > m_run[0] + kLazyMax || lm[1] > m_run[1] + kLazyMax) != 0) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const float m_new = fmaxf(m_run[nb], max_across_groups(lm[nb]));
        const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[nb] - m_new);
        m_run[nb] = m_new;
        l_lane[nb] *= alpha;
#pragma unroll
        for (int nd = 0; nd < ND; ++nd) acc[nd][nb] *= alpha;
      }
    }
    u32x4 pop[2][2];  // [key chunk of 32][row block]
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      // P = 2^(s * scale_log2 - m) in one FMA + exp; a row with no score yet gives P = 0.
      const float neg_m = m_run[nb] == -INFINITY ? 0.f : -m_run[nb];
      uint16_t ph[4][4];
      float sum = 0.f;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = fast_exp2(__builtin_fmaf(s[mb][nb][r], a.scale_log2, neg_m));
          sum += p;
          ph[mb][r] = f32_to_f16(p);
        }
      }
      l_lane[nb] += sum;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        pop[kc][nb] = u32x4{pack2(ph[2 * kc][0], ph[2 * kc][1]), pack2(ph[2 * kc][2], ph[2 * kc][3]),
                            pack2(ph[2 * kc + 1][0], ph[2 * kc + 1][1]), pack2(ph[2 * kc + 1][2], ph[2 * kc + 1][3])};
      }
    }
    // O^T[d][row] += V^T[d][key] P^T[key][row]
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int r0 = 32 * kc + tr_row;
        const int r1 = r0 + 16;
        const u32x2 lo = lds_read_tr16(vt + r0 * D + 8 * v_pos<D>(r0, 2 * nd + tr_chunk) + tr_half);
        const u32x2 hi = lds_read_tr16(vt + r1 * D + 8 * v_pos<D>(r1, 2 * nd + tr_chunk) + tr_half);
        const u32x4 vop = u32x4{lo[0], lo[1], hi[0], hi[1]};
        acc[nd][0] = mfma_16x16x32<kFloat16>(vop, pop[kc][0], acc[nd][0]);
        acc[nd][1] = mfma_16x16x32<kFloat16>(vop, pop[kc][1], acc[nd][1]);
      }
    }
  };

  if (n_kb > 0) {
    load_block(0);
    store_block(0, 0);
  }
  __syncthreads();
  for (int kb = 0; kb < n_kb; ++kb) {
    const bool more = kb + 1 < n_kb;
    if (more) load_block(kb + 1);  // in flight while this block is computed
    if (kb * kBlockN < wave_end) compute_block(kb, kb & 1);
    if (more) store_block(kb + 1, (kb + 1) & 1);
    __syncthreads();
  }

#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float l = sum_across_groups(l_lane[nb]);
    if (!row_ok[nb]) continue;
    const float inv = 1.f / l;
    const int pos = (32 * wave + 16 * nb + col) / GS;
    uint16_t* orow = a.out + static_cast<int64_t>(qs + m0 + pos) * a.o_st + static_cast<int64_t>(head[nb]) * a.o_sh;
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
static int launch_prefill(const PrefillArgs& a, int num_programs, hipStream_t stream) {
  using Shape = PrefillShape<GS>;
  const int64_t units = static_cast<int64_t>(num_programs) * Shape::kSub * a.kvg;
  if (units > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((paged_prefill_kernel<DT, D, GS>), dim3(static_cast<unsigned>(units)), dim3(Shape::kThreads), 0,
                     stream, a);
  return static_cast<int>(hipGetLastError());
}

template <int DT, int D>
static int dispatch_gs(const PrefillArgs& a, int gs, int num_programs, hipStream_t s) {
  switch (gs) {
    case 1:
      return launch_prefill<DT, D, 1>(a, num_programs, s);
    case 2:
      return launch_prefill<DT, D, 2>(a, num_programs, s);
    case 4:
      return launch_prefill<DT, D, 4>(a, num_programs, s);
    default:
      return launch_prefill<DT, D, 8>(a, num_programs, s);
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
  // Heads per unit: the largest of 8, 4, 2, 1 that divides G.
  const int gs = G % 8 == 0 ? 8 : (G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1));
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
  a.kvg = num_kv_heads * a.gsplit;
  a.scale_log2 = scale * 1.4426950408889634f;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kFloat16) {
    return head_dim == 64 ? dispatch_gs<kFloat16, 64>(a, gs, num_programs, s)
                          : dispatch_gs<kFloat16, 128>(a, gs, num_programs, s);
  }
  return head_dim == 64 ? dispatch_gs<kBFloat16, 64>(a, gs, num_programs, s)
                        : dispatch_gs<kBFloat16, 128>(a, gs, num_programs, s);
}
