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
// Each wave then computes, for its 32 rows (lane l: row l % 32, lanes l and
// l + 32 holding different keys of it):
//   S^T[key][row] = K[key][:] . Q^T[:][row]   32x32x16 MFMA, K read from LDS
//                                              in the A-operand layout, Q^T in
//                                              registers
//   softmax in the exp2 domain with a lazily raised running max: the max
//   only moves when a score exceeds it by more than 2^8, so the rescale of
//   O is rare and P = 2^(s - m) stays below 256 (exact range in fp16); row
//   sums stay per lane until the end
//   O^T[d][row]  += V^T[d][key] . P^T[key][row]  32x32x16 fp16 MFMA, V^T read
//                                              with ds_read_b64_tr_b16, P^T is
//                                              the QK output layout as is
// Causal and context masks are applied only on blocks that need them.
//
// Key-range pieces (nimbus_paged_prefill_pieces). When a batch has too few
// tiles to fill the chip, the heaviest tile's serial walk over its key
// blocks sets the time. The host then cuts heavy tiles' key ranges into
// pieces [kb0, kb1) of about equal length; a piece writes its rows'
// unnormalised fp32 O with the running max m and row sum l to a workspace
// slot, and paged_prefill_merge_kernel combines a tile's pieces with
// o = sum_i O_i 2^(m_i - M) / sum_i l_i 2^(m_i - M), M = max m_i (the rule
// decode's split pieces use).
#include <type_traits>

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
  const int32_t* pieces;  // [units][5]: seq, m0, kb0, kb1, slot (-1: whole); null: the plain tile table
  float* part;            // workspace: per slot [64 positions][H] rows of D floats of O, then (m, l) pairs
  int64_t part_ml;        // float offset of the (m, l) pairs: slots * 64 * H * D
  int32_t slots;          // workspace slots (a piece's slot at or past it is not written)
  uint16_t* out;
  int64_t o_st, o_sh;
  int32_t H, G, gsplit, kvg;
  float scale_log2;
  // Stream-K plan (nimbus_paged_prefill_stream), null otherwise: the pieces
  // of share j are sk_piece[sk_start[j] .. sk_start[j + 1]), kSkFields int32
  // each; sk_part holds the split pieces' (O, m, l) per (share, kv-head group,
  // wave); sk_flag one word per (share, kv-head group, wave), 1 while that
  // slot holds a piece not yet folded in; sk_err is set when a wait gives up.
  const int32_t* sk_start;
  const int32_t* sk_piece;
  float* sk_part;
  int32_t* sk_flag;
  int32_t* sk_err;
  int32_t sk_shares;  // shares per kv-head group (the grid is sk_shares * kvg)
};

template <int GS>
struct PrefillShape {
  static constexpr int kPos = 128 / GS < kPrefillTile ? 128 / GS : kPrefillTile;  // positions per unit
  static constexpr int kRows = kPos * GS;
  static constexpr int kWaves = kRows / 32;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kSub = kPrefillTile / kPos;  // units per tile-table entry
};

// Waves per SIMD the register budget is sized for: two, except the
// two-wave workgroups of GS = 1 at D = 128, whose staging registers double.
template <int D, int GS>
struct PrefillOccupancy {
  static constexpr int kWavesPerEU = (GS == 1 && D == 128) ? 1 : 2;
};

// Swizzled 16-byte chunk positions of the LDS tiles. The 64 banks serve 256
// bytes per cycle: sixteen lanes of a ds_read_b128, thirty-two of a
// ds_read_b64_tr_b16. K rows are read sixteen at a time (one key per lane
// column, all lanes the same chunk) by the QK operand loads; the transposed V
// reads take eight rows and two adjacent chunks per 32 lanes. XOR-ing the
// chunk index with a function of the row puts those reads on distinct banks.
// At D = 128 a row is the 256 bytes; at D = 64 two rows share them (row parity
// picks the half), so the function skips the parity bit: K uses key bits
// 1-3, V bits 1-2 (chunk pairs).
template <int D>
__device__ __forceinline__ int k_pos(int key, int c) {
  return D == 128 ? c ^ (key & 15) : c ^ ((key >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int v_pos(int key, int c) {
  return D == 128 ? c ^ ((4 * key) & 12) : c ^ (4 * ((key >> 1) & 1));
}

// min(max(x, 0), 16) on a wave-uniform x, in scalar instructions: written
// plainly, the compiler forms the clamp as v_med3_i32 (a vector instruction)
// and copies the result back with v_readfirstlane.
__device__ __forceinline__ int scalar_clamp16(int x) {
  int r;
  asm("s_max_i32 %0, %1, 0\n\ts_min_i32 %0, %0, 16" : "=&s"(r) : "s"(x) : "scc");
  return r;
}

__device__ __forceinline__ int32_t scalar_load_i32(const int32_t* p, int i) {
  typedef const __attribute__((address_space(4))) int32_t* const_ptr;
  return ((const_ptr)(p))[i];
}

// Page ids of one 64-key block (four pages), range-checked.
struct BlockPages {
  int id[4];
};

// Key-block range and piece slot of a unit of the plain tile table: every
// block of the unit, written as a whole (no piece).
__constant__ int32_t kWholeUnit[3] = {0, INT32_MAX, -1};

typedef float f32x16 __attribute__((ext_vector_type(16)));

// 32x32x16 MFMA: a, b carry 8 16-bit elements each. Lane l holds A[m = l % 32]
// [k = 8 (l / 32) + t] and B[k = 8 (l / 32) + t][n = l % 32]; result element
// i of lane l is D[m = 8 (i / 4) + 4 (l / 32) + i % 4][n = l % 32].
template <int DT>
__device__ __forceinline__ f32x16 mfma_32x32x16(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (DT == kFloat16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
}

template <int N>
using IntC = std::integral_constant<int, N>;
template <bool B>
using BoolC = std::integral_constant<bool, B>;

// Stream-K plan (nimbus_paged_prefill_stream): piece record fields.
enum SkField : int { kSkSeq = 0, kSkM0, kSkKb0, kSkKb1, kSkSlot, kSkFixLo, kSkFixHi, kSkFields = 8 };
// Polls of a fix-up wait before it gives up and flags the call as failed
// (the contributors it waits on are lower-numbered workgroups, dispatched
// before it, so a wait ends unless the plan is inconsistent).
constexpr int kSkMaxPolls = 1 << 22;
// Stream-K workspace layout, the same for every plan: a flag word per (share,
// kv-head group, wave) for the most workgroups a call accepts, then an error
// word (in a 256-byte line of its own), then the split pieces' slots. Flags
// sized to the plan would let one plan's slots lie where another plan's
// flags do, so a workspace shared by calls with different plans would start
// a call with nonzero "flags" (stale partials), and a fix-up would fold in
// pieces not yet written.
constexpr int64_t kSkMaxWorkgroups = 2048;                 // shares x kv-head groups (two per CU: 1,024 CUs)
constexpr int64_t kSkFlagBytes = kSkMaxWorkgroups * 4 * 4;  // four waves a workgroup at most, a word each

// SK: the workgroup walks the pieces of its stream-K share (one kv-head
// group, the share's list of (unit, key-block range) pieces); otherwise it
// is one unit of the tile table or of a key-range piece table.
// The kernel's argument block, read through the kernel-argument segment
// (the kernels' only argument sits at its start).
typedef const __attribute__((address_space(4))) PrefillArgs* ArgsPtr;
__device__ __forceinline__ ArgsPtr kernel_args() {
  return (ArgsPtr)(__builtin_amdgcn_kernarg_segment_ptr());
}

template <int DT, int D, int GS, bool SK>
__device__ __forceinline__ void prefill_unit() {
  ArgsPtr a_top = kernel_args();
  using Shape = PrefillShape<GS>;
  constexpr int NT = Shape::kThreads;
  constexpr int POS = Shape::kPos;
  constexpr int KK = D / 16;                // 32x32x16 steps over the head dim (QK)
  constexpr int ND = D / 32;                // 32-row blocks of O^T
  constexpr int CPR = D / 8;                // 16-byte chunks per K/V row
  constexpr int PPT = kBlockN * CPR / NT;   // 16-byte pieces per thread per tile
  constexpr int TILE = kBlockN * D;         // u16 elements of one tile
  constexpr int KPW = 64 / CPR;             // keys one wave's 64 lanes cover per piece
  constexpr int KSTEP = NT / CPR;           // keys between a thread's consecutive pieces
  static_assert((kBlockN * CPR) % NT == 0 && 16 % KPW == 0, "tile pieces must divide evenly");
  __shared__ __attribute__((aligned(16))) uint16_t ks[2 * TILE];
  __shared__ __attribute__((aligned(16))) uint16_t vs[2 * TILE];

  // Unit: kv-head group fastest, then the sub-tile, then the table entry
  // (stream-K: kv-head group fastest, then the share).
  const int kvg_id = blockIdx.x % a_top->kvg;
  const int r_unit = blockIdx.x / a_top->kvg;
  const int kvh = kvg_id / a_top->gsplit;
  const int gsub = kvg_id % a_top->gsplit;

  int p_first = 0, p_end = 1;
  if constexpr (SK) {
    p_first = scalar_load_i32(a_top->sk_start, r_unit);
    p_end = scalar_load_i32(a_top->sk_start, r_unit + 1);
  }
  for (int pc = p_first; pc < p_end; ++pc) {
  // Stream-K reads the arguments again for each piece (through a pointer the
  // compiler cannot see through): kept in scalar registers across the walk,
  // they would crowd out the walk's own.
  ArgsPtr ap = kernel_args();
  if constexpr (SK) {
    asm volatile("" : "+s"(ap));
    if (pc > p_first) __syncthreads();  // the previous piece's last LDS reads are done
  }
  const auto& a = *ap;
  // The unit's record (sequence, first query, key blocks [kb0, kb1), piece
  // slot), read without a branch: the plain tile table takes its block range
  // and slot from kWholeUnit. Before the first K/V copy the workgroup then
  // waits on three dependent rounds of scalar loads: the kernel arguments,
  // the record, and the sequence's bounds together with the page ids of its
  // first three key blocks (indexed from kb0 and clamped to the table row, so
  // they need no context length; a page past the context is read through an
  // empty buffer resource, whatever id its table entry holds).
  // (each empty asm below takes the values of one round, so the compiler
  // issues that round's loads together and none of them later)
  asm volatile("" ::"s"(a.pieces), "s"(a.prog_seq), "s"(a.prog_m), "s"(a.bt), "s"(a.bt_sb), "s"(a.qstart),
               "s"(a.ctx), "s"(a.q), "s"(a.kc), "s"(a.vc), "s"(a.c_sb), "s"(a.c_st), "s"(a.c_sh));
  int seq, m_entry, kb0, kb1, slot, fix_lo = 0, fix_hi = 0;
  const int entry = r_unit / Shape::kSub;
  const int sub = r_unit % Shape::kSub;
  if constexpr (SK) {
    const int32_t* rec = a.sk_piece + kSkFields * pc;
    seq = scalar_load_i32(rec, kSkSeq);
    m_entry = scalar_load_i32(rec, kSkM0);
    kb0 = scalar_load_i32(rec, kSkKb0);
    kb1 = scalar_load_i32(rec, kSkKb1);
    slot = scalar_load_i32(rec, kSkSlot);
    fix_lo = scalar_load_i32(rec, kSkFixLo);
    fix_hi = scalar_load_i32(rec, kSkFixHi);
    asm volatile("" : "+s"(seq), "+s"(m_entry), "+s"(kb0), "+s"(kb1), "+s"(slot), "+s"(fix_lo), "+s"(fix_hi));
  } else {
    const int32_t* p_rec = a.pieces ? a.pieces + 5 * entry : a.prog_seq + entry;
    const int32_t* p_m = a.pieces ? p_rec + 1 : a.prog_m + entry;
    const int32_t* p_blk = a.pieces ? p_rec + 2 : kWholeUnit;
    seq = scalar_load_i32(p_rec, 0);
    m_entry = scalar_load_i32(p_m, 0);
    kb0 = scalar_load_i32(p_blk, 0);
    kb1 = scalar_load_i32(p_blk, 1);
    slot = scalar_load_i32(p_blk, 2);
    asm volatile("" : "+s"(seq), "+s"(m_entry), "+s"(kb0), "+s"(kb1), "+s"(slot));
  }
  kb0 = max(kb0, 0);  // (a piece's first block; the page ids below are indexed from it)
  const int32_t* btrow = a.bt + seq * a.bt_sb;
  const int page_cap = a.bt_width - 1;
  auto load_raw = [&](int blk) {
    BlockPages p;
#pragma unroll
    for (int i = 0; i < 4; ++i) p.id[i] = scalar_load_i32(btrow, min(4 * blk + i, page_cap));
    return p;
  };
  auto checked = [&](BlockPages p) {
#pragma unroll
    for (int i = 0; i < 4; ++i) p.id[i] = static_cast<uint32_t>(p.id[i]) < static_cast<uint32_t>(a.num_blocks) ? p.id[i] : 0;
    return p;
  };
  auto load_pages = [&](int blk) { return checked(load_raw(blk)); };
  int qs = scalar_load_i32(a.qstart, seq);
  int qe = scalar_load_i32(a.qstart, seq + 1);
  int ctx_in = scalar_load_i32(a.ctx, seq);
  BlockPages pg_first = load_raw(kb0);
  BlockPages pg_v = load_raw(kb0 + 1);  // pages of V(kb + 1)
  BlockPages pg_k = load_raw(kb0 + 2);  // pages of K(kb + 2)
  // (the compiler would otherwise sink these past the exit below, or check
  // each page id as it lands and reuse its register: rounds of their own)
  asm volatile("" : "+s"(qs), "+s"(qe), "+s"(ctx_in), "+s"(pg_first.id[0]), "+s"(pg_first.id[1]),
               "+s"(pg_first.id[2]), "+s"(pg_first.id[3]), "+s"(pg_v.id[0]), "+s"(pg_v.id[1]), "+s"(pg_v.id[2]),
               "+s"(pg_v.id[3]), "+s"(pg_k.id[0]), "+s"(pg_k.id[1]), "+s"(pg_k.id[2]), "+s"(pg_k.id[3]));
  pg_first = checked(pg_first);
  pg_v = checked(pg_v);
  pg_k = checked(pg_k);
  const int m0 = SK ? m_entry : m_entry + sub * POS;
  const int q_len = qe - qs;
  if (m0 >= q_len) {  // the whole workgroup: this sub-tile has no queries (nor has it for any other piece of it)
    if constexpr (SK) continue;
    else return;
  }
  const int ctx = min(ctx_in, a.bt_width * 16);
  const int base_pos = ctx - q_len;  // absolute position of query 0
  const int kv_end = max(0, min(ctx, base_pos + m0 + POS));
  // This unit's key blocks [kbeg, kend): all of them, or its piece's share.
  const int n_kb_all = (kv_end + kBlockN - 1) / kBlockN;
  const int kbeg = min(kb0, n_kb_all);
  const int kend = min(kb1, n_kb_all);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64) & (Shape::kWaves - 1);  // scalar, range known
  const int lane = tid % 64;
  const int col = lane % 32;  // this lane's row of the wave's 32
  const int kg = lane / 32;   // which of each 16-long k range it holds (8 kg .. 8 kg + 7)

  // This lane's row (lanes l and l + 32 share it).
  int qpos, head;
  {
    const int r = 32 * wave + col;
    qpos = base_pos + m0 + r / GS;
    head = kvh * a.G + gsub * GS + r % GS;
  }
  // Smallest position among this wave's rows: blocks wholly at or below it
  // (and inside the context) need no mask.
  const int wave_lo = base_pos + m0 + (32 * wave) / GS;

  // Q^T as the B operand (rows past q_len load the last query row).
  u32x4 qop[KK];
  {
    const int pos = min((32 * wave + col) / GS, q_len - 1 - m0);
    const uint16_t* qrow = a.q + static_cast<int64_t>(qs + m0 + pos) * a.q_st + static_cast<int64_t>(head) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qop[kk] = *reinterpret_cast<const u32x4*>(qrow + 16 * kk + 8 * kg);
  }
  // ---- staging
  // Piece i of thread t is key lkey + KSTEP i, 16-byte slot lc of that LDS
  // row. All of a wave's lanes fall in one page for a given i, so each load
  // goes through a buffer resource (scalar registers) holding that page's
  // address, plus a fixed 32-bit per-lane offset. The resource's size is the
  // page's rows below kv_end, so keys past the context (in the last page, or
  // in pages of a block beyond it) read as zeros: P is 0 there, and 0 * 0
  // keeps garbage out of O. K goes global -> LDS directly
  // (buffer_load_dwordx4 ... lds: lane l's 16 bytes land at the wave's LDS
  // base + 16 l), so each lane loads the chunk that the swizzle puts in its
  // slot. fp16 V goes the same way; bf16 V passes through registers for
  // the fp16 conversion.
  const char* kbytes = reinterpret_cast<const char*>(a.kc + static_cast<int64_t>(kvh) * a.c_sh);
  const char* vbytes = reinterpret_cast<const char*>(a.vc + static_cast<int64_t>(kvh) * a.c_sh);
  const uint32_t page_bytes = static_cast<uint32_t>(a.c_sb * 2);  // below 2^31 (host check)
  const int row_bytes = static_cast<int>(a.c_st * 2);
  const int lkey = tid / CPR;
  const int lc = tid % CPR;
  int k_goff[PPT], v_goff[PPT], v_st[PPT];
#pragma unroll
  for (int i = 0; i < PPT; ++i) {
    const int key = lkey + KSTEP * i;
    k_goff[i] = (key % 16) * row_bytes + 16 * k_pos<D>(key, lc);  // k_pos is an involution in the chunk index
    // (converting bf16 V in place in LDS instead measured slower)
    v_goff[i] = (key % 16) * row_bytes + 16 * (DT == kFloat16 ? v_pos<D>(key, lc) : lc);  // v_pos is an involution too
    v_st[i] = key * D + 8 * v_pos<D>(key, lc);
  }
  // Buffer resource of the page holding piece i of this wave in block blk.
  auto page_rsrc = [&](const char* base, const BlockPages& p, int blk, int i) {
    const int j = (wave * KPW + KSTEP * i) / 16;
    // (readfirstlane on each id keeps the select from being folded into an
    // indexed load, which would put the ids in scratch memory)
    const int p0 = __builtin_amdgcn_readfirstlane(p.id[0]), p1 = __builtin_amdgcn_readfirstlane(p.id[1]);
    const int p2 = __builtin_amdgcn_readfirstlane(p.id[2]), p3 = __builtin_amdgcn_readfirstlane(p.id[3]);
    const int id = (j & 2) ? ((j & 1) ? p3 : p2) : ((j & 1) ? p1 : p0);
    const int rows = scalar_clamp16(kv_end - 16 * (4 * blk + j));
    // ids are checked nonnegative: a 32 x 32 -> 64-bit product
    const uint64_t off = static_cast<uint64_t>(static_cast<uint32_t>(id)) * page_bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + off, 0, rows * row_bytes, kBufferFlags);
  };
  typedef __attribute__((address_space(3))) void lds_void;
  auto dma_k = [&](const BlockPages& p, int blk, auto slot) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      uint16_t* dst = ks + slot * TILE + (wave * KPW + KSTEP * i) * D;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(page_rsrc(kbytes, p, blk, i), (lds_void*)dst, 16, k_goff[i], 0, 0, 0);
    }
  };
  u32x4 vreg[DT == kFloat16 ? 1 : PPT];
  // V(blk) into LDS slot `slot`: issued here, completed by store_v.
  auto issue_v = [&](const BlockPages& p, int blk, auto slot) {
#pragma unroll
    for (int i = 0; i < PPT; ++i) {
      if constexpr (DT == kFloat16) {
        uint16_t* dst = vs + slot * TILE + (wave * KPW + KSTEP * i) * D;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(page_rsrc(vbytes, p, blk, i), (lds_void*)dst, 16, v_goff[i], 0, 0,
                                                 0);
      } else {
        vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(page_rsrc(vbytes, p, blk, i), v_goff[i], 0, 0);
      }
    }
  };
  auto store_v = [&](auto slot) {
    if constexpr (DT == kBFloat16) {
#pragma unroll
      for (int i = 0; i < PPT; ++i) {
        u32x4 v = vreg[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = v_to_f16_pair<DT>(v[e]);
        *reinterpret_cast<u32x4*>(vs + slot * TILE + v_st[i]) = v;
      }
    }
  };

  // ---- per-wave math
  // S^T of one block, per 32-key half h: element i of lane l is key
  // 32 h + 8 (i / 4) + 4 kg + i % 4 of the block, row col.
  typedef f32x16 Scores[2];
  // Running max before a row has seen a key: finite, so the rescale factor
  // 2^(m_run - m_new) and the exponent s * scale_log2 - m_run need no -inf
  // case (a masked score stays -inf; the first visible score always moves the
  // max, before any P of its block is formed). Lanes l and l + 32 keep the
  // same value for their shared row.
  constexpr float kNoMax = -0x1p127f;
  float m_run = kNoMax;
  f32x16 acc[ND];  // O^T: element i of lane l is d = 32 nd + 8 (i / 4) + 4 kg + i % 4, row col
  float lsum = 0.f;  // this lane's share of its row's sum of the fp16 P (the keys it holds)
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[nd][i] = 0.f;
  }
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 ones2 = h2{static_cast<_Float16>(1.f), static_cast<_Float16>(1.f)};

  // S^T[key][row] = K[key][:] . Q^T[:][row] for keys 32 h .. 32 h + 31.
  auto qk = [&](auto slot, auto half, Scores& s) {
    constexpr int H = decltype(half)::value;
    const uint16_t* kt = ks + slot * TILE;
    const int key = 32 * H + col;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[H][i] = 0.f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u32x4 kop = *reinterpret_cast<const u32x4*>(kt + key * D + 8 * k_pos<D>(key, 2 * kk + kg));
      s[H] = mfma_32x32x16<DT>(kop, qop[kk], s[H]);
    }
  };
  // Mask (raw scores; only blocks that reach past a row's position or the
  // context need it), then the lazy running max (exp2 domain): it moves, and
  // O and the row sums are rescaled, only when a score is more than
  // 2^kLazyMax above it, so P <= 2^kLazyMax.
  auto mask_and_max = [&](Scores& s, int blk) {
    const int k0 = blk * kBlockN;
    const bool full = k0 + kBlockN - 1 <= wave_lo && k0 + kBlockN <= kv_end;
    if (!full) {
      const int lim = min(qpos + 1, kv_end) - k0 - 4 * kg;  // key offsets below lim are visible
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int i = 0; i < 16; ++i) s[h][i] = 32 * h + 8 * (i / 4) + i % 4 < lim ? s[h][i] : -INFINITY;
      }
    }
    float m = -INFINITY;  // (a constant start spares the canonicalising max of the first score)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int i = 0; i < 16; ++i) m = fmaxf(m, s[h][i]);
    }
    const float lm = m * a.scale_log2;  // the scale is positive: max commutes with it
    if (__builtin_amdgcn_ballot_w64(lm > m_run + kLazyMax) != 0) {
      const float m_new = fmaxf(m_run, fmaxf(lm, __shfl_xor(lm, 32, 64)));
      const float alpha = fast_exp2(m_run - m_new);
      m_run = m_new;
      lsum *= alpha;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) acc[nd] *= alpha;
    }
  };
  // P^T = 2^(S^T * scale_log2 - m) for keys 32 h .. 32 h + 31 as the fp16 B
  // operands of the two P.V MFMAs (keys 32 h + 16 j ..); a row with no score
  // yet gives P = 0. Operand element t (k = 8 kg + t) is S element 8 j + t,
  // key 32 h + 16 j + 8 (t / 4) + 4 kg + t % 4.
  auto probs = [&](const Scores& s, auto half, u32x4 (&pop)[2]) {
    constexpr int H = decltype(half)::value;
    const float neg_m = -m_run;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      float p[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) p[t] = fast_exp2(__builtin_fmaf(s[H][8 * j + t], a.scale_log2, neg_m));
      pop[j] = u32x4{pack_f16_rtz(p[0], p[1]), pack_f16_rtz(p[2], p[3]), pack_f16_rtz(p[4], p[5]),
                     pack_f16_rtz(p[6], p[7])};
    }
  };
  // Transposed-read addresses (see lds_read_tr16): in each 16-lane group
  // (kg = group / 2, column half group % 2), lane i reads V row
  // 32 h + 16 j + 4 kg + i / 4 (and + 8), elements
  // 32 nd + 16 (group % 2) + 4 (i % 4) .. +4; lane i of the group then holds
  // d = 32 nd + 16 (group % 2) + i, the A operand's row l % 32.
  const int gi = lane % 16;
  const int tr_row = 4 * kg + gi / 4;
  const int tr_chunk = 2 * ((lane / 16) % 2) + (gi % 4) / 2;
  const int tr_half = 4 * ((gi % 4) % 2);
  // O^T[d][row] += V^T[d][key] P^T[key][row] for keys 32 h .. 32 h + 31; the
  // lane's row-sum share += its P.
  auto pv = [&](auto slot, auto half, const u32x4 (&pop)[2]) {
    constexpr int H = decltype(half)::value;
    const uint16_t* vt = vs + slot * TILE;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int r0 = 32 * H + 16 * j + tr_row;
      const int r1 = r0 + 8;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
        const u32x2 lo = lds_read_tr16(vt + r0 * D + 8 * v_pos<D>(r0, 4 * nd + tr_chunk) + tr_half);
        const u32x2 hi = lds_read_tr16(vt + r1 * D + 8 * v_pos<D>(r1, 4 * nd + tr_chunk) + tr_half);
        const u32x4 vop = u32x4{lo[0], lo[1], hi[0], hi[1]};
        acc[nd] = mfma_32x32x16<kFloat16>(vop, pop[j], acc[nd]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = pop[j][e];  // (a bit_cast of the vector subscript itself would read element 0)
        lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, w), ones2, lsum, false);
      }
    }
  };

  // ---- the block pipeline
  // Iteration kb: the K tile of block kb + 1 and the V tile of block kb are
  // in LDS (slots (kb + 1) & 1 and kb & 1), and S of block kb in registers.
  // It issues the loads of V(kb + 1) and K(kb + 2), the latter straight into
  // the slot K(kb) left (last read before the previous barrier); then, for
  // each 32-key half, computes P(kb) while the QK products of block kb + 1
  // run, and P(kb).V(kb); then it stores V(kb + 1) into the slot V(kb - 1)
  // left, masks and takes the max of S(kb + 1), and meets the other waves at
  // one barrier, which also waits for the K copies. The page ids of a block
  // are read one iteration before its loads are issued.
  Scores sa, sb;
  if (kend > kbeg) {  // (then kbeg = kb0)
    issue_v(pg_first, kbeg, IntC<0>{});
    dma_k(pg_first, kbeg, IntC<0>{});
    // K(kbeg + 1) goes with the first block's loads (slot 1 is free), so the
    // first barrier waits for both at once. Past the context it reads zeros;
    // past the piece it is never read.
    dma_k(pg_v, kbeg + 1, IntC<1>{});
    __syncthreads();
    qk(IntC<0>{}, IntC<0>{}, sa);
    qk(IntC<0>{}, IntC<1>{}, sa);
    store_v(IntC<0>{});
    mask_and_max(sa, kbeg);
    __syncthreads();
  }
  // Two forms of the iteration: with the next block (all but the last) and
  // the last one. The first form always issues K(kb + 2): past the context
  // it reads zeros through an empty buffer resource, past a piece's range it
  // is loaded and never read. So the walk inlines five copies of the
  // iteration in two forms instead of one per tail length and form, which
  // keeps the tail inside the register budget.
  auto iteration = [&](int kb, auto slot, auto has_next, Scores& s_cur, Scores& s_nxt) {
    constexpr int SLOT = decltype(slot)::value;
    constexpr bool NEXT = decltype(has_next)::value;
    BlockPages pg_n;
    if constexpr (NEXT) {
      issue_v(pg_v, kb + 1, IntC<1 - SLOT>{});
      pg_n = load_pages(kb + 3);
      dma_k(pg_k, kb + 2, IntC<SLOT>{});
    }
    {
      u32x4 pop[2];
      probs(s_cur, IntC<0>{}, pop);
      if constexpr (NEXT) qk(IntC<1 - SLOT>{}, IntC<0>{}, s_nxt);
      pv(IntC<SLOT>{}, IntC<0>{}, pop);
    }
    {
      u32x4 pop[2];
      probs(s_cur, IntC<1>{}, pop);
      if constexpr (NEXT) qk(IntC<1 - SLOT>{}, IntC<1>{}, s_nxt);
      pv(IntC<SLOT>{}, IntC<1>{}, pop);
    }
    if constexpr (NEXT) {
      store_v(IntC<1 - SLOT>{});
      mask_and_max(s_nxt, kb + 1);
      __syncthreads();
      pg_v = pg_k;
      pg_k = pg_n;
    }
  };
  int kb = kbeg;
  for (; kb + 2 < kend; kb += 2) {
    iteration(kb, IntC<0>{}, BoolC<true>{}, sa, sb);
    iteration(kb + 1, IntC<1>{}, BoolC<true>{}, sb, sa);
  }
  // kb - kbeg is even here; one or two iterations remain.
  if (kb + 1 < kend) {
    iteration(kb, IntC<0>{}, BoolC<true>{}, sa, sb);
    iteration(kb + 1, IntC<1>{}, BoolC<false>{}, sb, sa);
  } else if (kb < kend) {
    iteration(kb, IntC<0>{}, BoolC<false>{}, sa, sb);
  }
  // The last K copies issued may still be in flight (into a slot nothing
  // reads any more); let them land before the workgroup's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // The output row's head and bound again, from a copy of the lane index
  // the compiler cannot see through: keeping the prologue's values alive
  // across the walk would cost registers the walk needs.
  int lane_e = lane;
  asm volatile("" : "+v"(lane_e));
  const int col_e = lane_e % 32;
  const int kg_e = lane_e / 32;
  const int r_e = 32 * wave + col_e;
  const bool row_ok = m0 + r_e / GS < q_len;
  const int head_e = kvh * a.G + gsub * GS + r_e % GS;

  if constexpr (SK) {
    // A stream-K piece. Its (O, m, l) live in a slot of the workspace per
    // (share, kv-head group, wave), one f32x4 per (row block, quad) and lane
    // and an (m, lsum) pair per lane: the lane layout of the registers, so
    // that the workgroup finishing the unit reads back exactly its own lanes.
    // The slot is written and read with agent-scope (sc1) accesses, which
    // bypass the non-coherent L2 of the writer's and reader's XCDs; the
    // writer's flag for (slot, wave) goes out once its stores are complete.
    constexpr int SLOT_FLOATS = (ND * 16 + 2) * 64;  // per wave
    auto slot_rsrc = [&](int s) {
      float* base = a.sk_part + (static_cast<int64_t>(s) * Shape::kWaves + wave) * SLOT_FLOATS;
      return __builtin_amdgcn_make_buffer_rsrc(base, 0, SLOT_FLOATS * 4, kBufferFlags);
    };
    if (slot >= 0) {
      if (slot >= a.sk_shares) continue;  // (a plan outside its workspace: nothing is written)
      const int s = slot * a.kvg + kvg_id;
      const auto rs = slot_rsrc(s);
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 v = f32x4{acc[nd][4 * q4], acc[nd][4 * q4 + 1], acc[nd][4 * q4 + 2], acc[nd][4 * q4 + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, ((nd * 4 + q4) * 64 + lane_e) * 16,
                                                 0, kSc1);
        }
      }
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(m_run), __float_as_uint(lsum)}, rs,
                                            (ND * 16 * 64 + 2 * lane_e) * 4, 0, kSc1);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      if (lane_e == 0) __hip_atomic_store(a.sk_flag + s * Shape::kWaves + wave, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
      continue;
    }
    // The unit's last piece: fold in the pieces of the lower-numbered shares
    // [fix_lo, fix_hi) (each wave its own rows), then write the output.
    // (only shares below this one: whatever the plan holds, a wait is on a
    // workgroup dispatched earlier)
    const int c_end = min(fix_hi, r_unit);
    for (int c = max(fix_lo, 0); c < c_end; ++c) {
      const int s = c * a.kvg + kvg_id;
      int32_t* flag = a.sk_flag + s * Shape::kWaves + wave;
      for (int polls = 0;; ++polls) {
        const int f = __builtin_amdgcn_readfirstlane(__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (f != 0) break;
        if (polls >= kSkMaxPolls) {
          if (lane_e == 0) __hip_atomic_store(a.sk_err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      asm volatile("" ::: "memory");
      const auto rs = slot_rsrc(s);
      const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(rs, (ND * 16 * 64 + 2 * lane_e) * 4, 0, kSc1);
      f32x4 po[ND * 4];
#pragma unroll
      for (int i = 0; i < ND * 4; ++i)
        po[i] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (i * 64 + lane_e) * 16, 0, kSc1));
      if (lane_e == 0) __hip_atomic_store(flag, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // for the next call
      const float m_c = __uint_as_float(ml[0]);
      const float m_new = fmaxf(m_run, m_c);
      const float a_own = fast_exp2(m_run - m_new), a_c = fast_exp2(m_c - m_new);
      m_run = m_new;
      lsum = lsum * a_own + __uint_as_float(ml[1]) * a_c;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[nd][i] = acc[nd][i] * a_own + po[nd * 4 + i / 4][i % 4] * a_c;
      }
    }
    if (row_ok) {
      const float inv = 1.f / (lsum + __shfl_xor(lsum, 32, 64));
      const int pos = r_e / GS;
      uint16_t* orow =
          a.out + static_cast<int64_t>(qs + m0 + pos) * a.o_st + static_cast<int64_t>(head_e) * a.o_sh;
#pragma unroll
      for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x16& o = acc[nd];
          const u32x2 w =
              u32x2{pack2(Elem<DT>::from_f32(o[4 * q4] * inv), Elem<DT>::from_f32(o[4 * q4 + 1] * inv)),
                    pack2(Elem<DT>::from_f32(o[4 * q4 + 2] * inv), Elem<DT>::from_f32(o[4 * q4 + 3] * inv))};
          *reinterpret_cast<u32x2*>(orow + 32 * nd + 8 * q4 + 4 * kg_e) = w;
        }
      }
    }
    continue;
  } else {
  const float l_row = lsum + __shfl_xor(lsum, 32, 64);  // both halves of the row's keys

  if (slot >= 0) {
    if (slot >= a.slots) return;
    // A piece: unnormalised O^T, the running max and the row sum, per row
    // (rows past q_len are skipped; a row that saw no key here writes
    // m = -inf, l = 0, O = 0 and weighs nothing in the merge).
    if (!row_ok) return;
    const int pos = m0 - m_entry + r_e / GS;
    const int64_t row = (static_cast<int64_t>(slot) * kPrefillTile + pos) * a.H + head_e;
    float* po = a.part + row * D;
#pragma unroll
    for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        *reinterpret_cast<f32x4*>(po + 32 * nd + 8 * q4 + 4 * kg_e) =
            f32x4{acc[nd][4 * q4], acc[nd][4 * q4 + 1], acc[nd][4 * q4 + 2], acc[nd][4 * q4 + 3]};
      }
    }
    if (kg_e == 0) {
      const float m_out = l_row == 0.f ? -INFINITY : m_run;
      *reinterpret_cast<float2*>(a.part + a.part_ml + row * 2) = make_float2(m_out, l_row);
    }
    return;
  }

  if (!row_ok) return;
  const float inv = 1.f / l_row;
  const int pos = r_e / GS;
  uint16_t* orow = a.out + static_cast<int64_t>(qs + m0 + pos) * a.o_st + static_cast<int64_t>(head_e) * a.o_sh;
#pragma unroll
  for (int nd = 0; nd < ND; ++nd) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x16& o = acc[nd];
      const u32x2 w = u32x2{pack2(Elem<DT>::from_f32(o[4 * q4] * inv), Elem<DT>::from_f32(o[4 * q4 + 1] * inv)),
                            pack2(Elem<DT>::from_f32(o[4 * q4 + 2] * inv), Elem<DT>::from_f32(o[4 * q4 + 3] * inv))};
      *reinterpret_cast<u32x2*>(orow + 32 * nd + 8 * q4 + 4 * kg_e) = w;
    }
  }
  }
  }  // pieces
}


template <int DT, int D>
__global__ __launch_bounds__(256) void paged_prefill_merge_kernel(PrefillArgs a, const int32_t* merges,
                                                                  int32_t num_merges) {
  constexpr int SEG = D / 8;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t per_tile = static_cast<int64_t>(kPrefillTile) * a.H * SEG;
  if (idx >= per_tile * num_merges) return;
  const int e = static_cast<int>(idx / per_tile);
  const int rem = static_cast<int>(idx % per_tile);
  const int pos = rem / (a.H * SEG);
  const int head = (rem / SEG) % a.H;
  const int d0 = 8 * (rem % SEG);
  const int32_t* me = merges + 4 * e;
  const int seq = me[0], m0 = me[1], slot0 = me[2], n = me[3];
  if (slot0 < 0 || n <= 0 || slot0 + n > a.slots) return;
  const int qs = a.qstart[seq];
  if (m0 + pos >= a.qstart[seq + 1] - qs) return;
  float M = -INFINITY;
  for (int i = 0; i < n; ++i) {
    const int64_t row = (static_cast<int64_t>(slot0 + i) * kPrefillTile + pos) * a.H + head;
    M = fmaxf(M, a.part[a.part_ml + row * 2]);
  }
  float L = 0.f, O[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) O[k] = 0.f;
  for (int i = 0; i < n; ++i) {
    const int64_t row = (static_cast<int64_t>(slot0 + i) * kPrefillTile + pos) * a.H + head;
    const float2 ml = *reinterpret_cast<const float2*>(a.part + a.part_ml + row * 2);
    const float w = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - M);
    const f32x4 o0 = *reinterpret_cast<const f32x4*>(a.part + row * D + d0);
    const f32x4 o1 = *reinterpret_cast<const f32x4*>(a.part + row * D + d0 + 4);
    L += ml.y * w;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      O[k] += o0[k] * w;
      O[k + 4] += o1[k] * w;
    }
  }
  const float inv = 1.f / L;
  uint16_t* orow = a.out + static_cast<int64_t>(qs + m0 + pos) * a.o_st + static_cast<int64_t>(head) * a.o_sh + d0;
  const u32x4 w4 = u32x4{pack2(Elem<DT>::from_f32(O[0] * inv), Elem<DT>::from_f32(O[1] * inv)),
                         pack2(Elem<DT>::from_f32(O[2] * inv), Elem<DT>::from_f32(O[3] * inv)),
                         pack2(Elem<DT>::from_f32(O[4] * inv), Elem<DT>::from_f32(O[5] * inv)),
                         pack2(Elem<DT>::from_f32(O[6] * inv), Elem<DT>::from_f32(O[7] * inv))};
  *reinterpret_cast<u32x4*>(orow) = w4;
}

// One kernel per register budget (the occupancy attribute takes a constant).
template <int DT, int D, int GS, bool SK>
__global__ __launch_bounds__(PrefillShape<GS>::kThreads) __attribute__((amdgpu_waves_per_eu(2))) void
paged_prefill_kernel(PrefillArgs) {
  prefill_unit<DT, D, GS, SK>();
}

template <int DT, int D, int GS, bool SK>
__global__ __launch_bounds__(PrefillShape<GS>::kThreads) __attribute__((amdgpu_waves_per_eu(1))) void
paged_prefill_kernel_1w(PrefillArgs) {
  prefill_unit<DT, D, GS, SK>();
}

template <int DT, int D>
static int launch_merge(const PrefillArgs& a, const int32_t* merges, int32_t num_merges, hipStream_t stream) {
  if (num_merges <= 0) return static_cast<int>(hipGetLastError());
  const int64_t threads = static_cast<int64_t>(num_merges) * kPrefillTile * a.H * (D / 8);
  hipLaunchKernelGGL((paged_prefill_merge_kernel<DT, D>), dim3(static_cast<unsigned>((threads + 255) / 256)),
                     dim3(256), 0, stream, a, merges, num_merges);
  return static_cast<int>(hipGetLastError());
}

// num_programs: tile-table entries (or pieces); stream-K: shares per kv-head
// group (a.sk_start set).
template <int DT, int D, int GS>
static int launch_prefill(const PrefillArgs& a, int num_programs, hipStream_t stream) {
  using Shape = PrefillShape<GS>;
  const int64_t units = static_cast<int64_t>(num_programs) * (a.sk_start ? 1 : Shape::kSub) * a.kvg;
  if (units > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<unsigned>(units)), block(Shape::kThreads);
  if constexpr (PrefillOccupancy<D, GS>::kWavesPerEU == 1) {
    if (a.sk_start) hipLaunchKernelGGL((paged_prefill_kernel_1w<DT, D, GS, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((paged_prefill_kernel_1w<DT, D, GS, false>), grid, block, 0, stream, a);
  } else {
    if (a.sk_start) hipLaunchKernelGGL((paged_prefill_kernel<DT, D, GS, true>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((paged_prefill_kernel<DT, D, GS, false>), grid, block, 0, stream, a);
  }
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

static int prefill_impl(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                        const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                        int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                        int64_t bt_stride, int32_t bt_width, const int32_t* query_start, const int32_t* context_lens,
                        const int32_t* prog_seq, const int32_t* prog_m, const int32_t* pieces, int32_t num_units,
                        const int32_t* merges, int32_t num_merges, int32_t num_slots, void* workspace,
                        int64_t workspace_bytes, void* out, int64_t out_stride_t, int64_t out_stride_h,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                        int32_t dtype, void* stream, const int32_t* sk_start = nullptr,
                        const int32_t* sk_piece = nullptr) {
  if (num_units < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  // Pages of other than 16 tokens and head dims other than 64 and 128 take
  // the general kernel (paged_general.hip), over the plain tile table.
  if (general_shape(head_dim, block_size)) {
    const int rc = general_check(head_dim, block_size);
    if (rc != 0) return rc;
    if (pieces || sk_start) return NIMBUS_ERR_UNSUPPORTED;
    if (num_units == 0) return NIMBUS_OK;
    if (!q || !k_cache || !v_cache || !block_tables || !query_start || !context_lens || !out || !prog_seq ||
        !prog_m)
      return NIMBUS_ERR_INVALID;
    if (num_blocks <= 0 || num_blocks > INT32_MAX || bt_width <= 0) return NIMBUS_ERR_INVALID;
    if (static_cast<int64_t>(bt_width) * block_size > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
    AttnGeneralArgs g{};
    g.q = static_cast<const uint16_t*>(q);
    g.q_st = q_stride_t;
    g.q_sh = q_stride_h;
    g.kc = static_cast<const uint16_t*>(k_cache);
    g.vc = static_cast<const uint16_t*>(v_cache);
    g.c_sb = cache_stride_block;
    g.c_st = cache_stride_token;
    g.c_sh = cache_stride_head;
    g.bt = block_tables;
    g.bt_sb = bt_stride;
    g.bt_width = bt_width;
    g.num_blocks = static_cast<int32_t>(num_blocks);
    g.bs = block_size;
    g.ctx = context_lens;
    g.qstart = query_start;
    g.prog_seq = prog_seq;
    g.prog_m = prog_m;
    g.tile_pos = kPrefillTile;
    g.out = static_cast<uint16_t*>(out);
    g.o_st = out_stride_t;
    g.o_sh = out_stride_h;
    g.H = num_heads;
    g.G = num_heads / num_kv_heads;
    g.KV = num_kv_heads;
    g.D = head_dim;
    g.scale_log2 = scale * 1.4426950408889634f;
    return launch_general_prefill(g, num_units, dtype, static_cast<hipStream_t>(stream));
  }
  const int G = num_heads / num_kv_heads;
  // Heads per unit: the largest of 8, 4, 2, 1 that divides G.
  const int gs = G % 8 == 0 ? 8 : (G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1));
  if (num_units == 0) return NIMBUS_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !query_start || !context_lens || !out) return NIMBUS_ERR_INVALID;
  if (!pieces && !sk_start && (!prog_seq || !prog_m)) return NIMBUS_ERR_INVALID;
  if (sk_start && !sk_piece) return NIMBUS_ERR_INVALID;
  if (num_blocks <= 0 || num_blocks > INT32_MAX || bt_width <= 0) return NIMBUS_ERR_INVALID;
  // Pages are read through buffer resources with 32-bit offsets: 16 token
  // rows of a page must span less than 2 GiB.
  if (cache_stride_token <= 0 || cache_stride_token > (int64_t{1} << 25)) return NIMBUS_ERR_UNSUPPORTED;
  // A page's byte offset is formed as page id x page bytes, in 32 x 32 bits.
  if (cache_stride_block <= 0 || cache_stride_block >= (int64_t{1} << 30)) return NIMBUS_ERR_UNSUPPORTED;
  if ((q_stride_t | q_stride_h | cache_stride_block | cache_stride_token | cache_stride_head | out_stride_t |
       out_stride_h) % 8 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
       reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if (pieces) {
    if (num_slots < 0 || num_merges < 0 || (num_merges > 0 && !merges)) return NIMBUS_ERR_INVALID;
    const int64_t need = static_cast<int64_t>(num_slots) * kPrefillTile * num_heads * (head_dim + 2) * 4;
    if (num_slots > 0 && (workspace == nullptr || workspace_bytes < need)) return NIMBUS_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return NIMBUS_ERR_ALIGNMENT;
  }

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
  a.pieces = pieces;
  a.part = static_cast<float*>(workspace);
  a.part_ml = static_cast<int64_t>(num_slots) * kPrefillTile * num_heads * head_dim;
  a.slots = pieces ? num_slots : 0;
  a.out = static_cast<uint16_t*>(out);
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  a.H = num_heads;
  a.G = G;
  a.gsplit = G / gs;
  a.kvg = num_kv_heads * a.gsplit;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.sk_start = sk_start;
  a.sk_piece = sk_piece;
  a.sk_part = nullptr;
  a.sk_flag = nullptr;
  a.sk_err = nullptr;
  a.sk_shares = 0;
  if (sk_start) {
    // num_units counts the shares per kv-head group; every workgroup of the
    // grid must be resident at once (two per CU).
    int64_t cus = 0;
    const int e = device_cus(&cus);
    if (e != 0) return e;
    if (static_cast<int64_t>(num_units) * a.kvg > 2 * cus ||
        static_cast<int64_t>(num_units) * a.kvg > kSkMaxWorkgroups)
      return NIMBUS_ERR_UNSUPPORTED;
    const int waves = gs == 1 ? 2 : 4;
    const int64_t slots = static_cast<int64_t>(num_units) * a.kvg * waves;
    const int64_t flag_bytes = kSkFlagBytes;
    const int64_t need = flag_bytes + 256 + slots * (head_dim / 32 * 16 + 2) * 64 * 4;
    if (workspace == nullptr || workspace_bytes < need) return NIMBUS_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0) return NIMBUS_ERR_ALIGNMENT;
    char* ws = static_cast<char*>(workspace);
    a.sk_flag = reinterpret_cast<int32_t*>(ws);
    a.sk_err = reinterpret_cast<int32_t*>(ws + flag_bytes);
    a.sk_part = reinterpret_cast<float*>(ws + flag_bytes + 256);
    a.sk_shares = num_units;
  }

  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc;
  if (dtype == kFloat16) {
    rc = head_dim == 64 ? dispatch_gs<kFloat16, 64>(a, gs, num_units, s)
                        : dispatch_gs<kFloat16, 128>(a, gs, num_units, s);
  } else {
    rc = head_dim == 64 ? dispatch_gs<kBFloat16, 64>(a, gs, num_units, s)
                        : dispatch_gs<kBFloat16, 128>(a, gs, num_units, s);
  }
  if (rc != 0 || !pieces || num_merges == 0) return rc;
  if (dtype == kFloat16) {
    return head_dim == 64 ? launch_merge<kFloat16, 64>(a, merges, num_merges, s)
                          : launch_merge<kFloat16, 128>(a, merges, num_merges, s);
  }
  return head_dim == 64 ? launch_merge<kBFloat16, 64>(a, merges, num_merges, s)
                        : launch_merge<kBFloat16, 128>(a, merges, num_merges, s);
}

extern "C" int nimbus_paged_prefill(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                    const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                    int64_t cache_stride_token, int64_t cache_stride_head,
                                    const int32_t* block_tables, int64_t bt_stride, int32_t bt_width,
                                    const int32_t* query_start, const int32_t* context_lens,
                                    const int32_t* prog_seq, const int32_t* prog_m, int32_t num_programs,
                                    void* out, int64_t out_stride_t, int64_t out_stride_h, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                    int32_t dtype, void* stream) {
  return prefill_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_blocks, cache_stride_block,
                      cache_stride_token, cache_stride_head, block_tables, bt_stride, bt_width, query_start,
                      context_lens, prog_seq, prog_m, nullptr, num_programs, nullptr, 0, 0, nullptr, 0, out,
                      out_stride_t, out_stride_h, num_heads, num_kv_heads, head_dim, block_size, scale, dtype, stream);
}

extern "C" int64_t nimbus_paged_prefill_pieces_workspace_bytes(int32_t num_slots, int32_t num_heads,
                                                               int32_t head_dim) {
  if (num_slots < 0 || num_heads <= 0 || head_dim <= 0) return -1;
  return static_cast<int64_t>(num_slots) * kPrefillTile * num_heads * (head_dim + 2) * 4;
}

extern "C" int nimbus_paged_prefill_pieces(const void* q, int64_t q_stride_t, int64_t q_stride_h, const void* k_cache,
                                           const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                                           int64_t cache_stride_token, int64_t cache_stride_head,
                                           const int32_t* block_tables, int64_t bt_stride, int32_t bt_width,
                                           const int32_t* query_start, const int32_t* context_lens,
                                           const int32_t* pieces, int32_t num_pieces, const int32_t* merges,
                                           int32_t num_merges, int32_t num_slots, void* workspace,
                                           int64_t workspace_bytes, void* out, int64_t out_stride_t,
                                           int64_t out_stride_h, int32_t num_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int32_t block_size, float scale, int32_t dtype,
                                           void* stream) {
  if (!pieces) return NIMBUS_ERR_INVALID;
  return prefill_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_blocks, cache_stride_block,
                      cache_stride_token, cache_stride_head, block_tables, bt_stride, bt_width, query_start,
                      context_lens, nullptr, nullptr, pieces, num_pieces, merges, num_merges, num_slots, workspace,
                      workspace_bytes, out, out_stride_t, out_stride_h, num_heads, num_kv_heads, head_dim,
                      block_size, scale, dtype, stream);
}

// Stream-K workspace: the flags (zero before the first call; every call that
// completes leaves them zero) and the error word, at the same offsets for
// every plan, then the split pieces' slots.
static int64_t stream_slots(int32_t shares, int32_t num_heads, int32_t num_kv_heads) {
  const int G = num_heads / num_kv_heads;
  const int gs = G % 8 == 0 ? 8 : (G % 4 == 0 ? 4 : (G % 2 == 0 ? 2 : 1));
  return static_cast<int64_t>(shares) * num_kv_heads * (G / gs) * (gs == 1 ? 2 : 4);
}

extern "C" int64_t nimbus_paged_prefill_stream_flag_bytes(int32_t num_shares, int32_t num_heads,
                                                          int32_t num_kv_heads) {
  if (num_shares < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return -1;
  return kSkFlagBytes + 256;
}

extern "C" int64_t nimbus_paged_prefill_stream_workspace_bytes(int32_t num_shares, int32_t num_heads,
                                                               int32_t num_kv_heads, int32_t head_dim) {
  const int64_t flags = nimbus_paged_prefill_stream_flag_bytes(num_shares, num_heads, num_kv_heads);
  if (flags < 0 || head_dim <= 0) return -1;
  return flags + stream_slots(num_shares, num_heads, num_kv_heads) * (head_dim / 32 * 16 + 2) * 64 * 4;
}

extern "C" int nimbus_paged_prefill_stream(const void* q, int64_t q_stride_t, int64_t q_stride_h,
                                           const void* k_cache, const void* v_cache, int64_t num_blocks,
                                           int64_t cache_stride_block, int64_t cache_stride_token,
                                           int64_t cache_stride_head, const int32_t* block_tables, int64_t bt_stride,
                                           int32_t bt_width, const int32_t* query_start,
                                           const int32_t* context_lens, const int32_t* share_start,
                                           const int32_t* pieces, int32_t num_shares, void* workspace,
                                           int64_t workspace_bytes, void* out, int64_t out_stride_t,
                                           int64_t out_stride_h, int32_t num_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int32_t block_size, float scale, int32_t dtype,
                                           void* stream) {
  if (!share_start || !pieces) return NIMBUS_ERR_INVALID;
  return prefill_impl(q, q_stride_t, q_stride_h, k_cache, v_cache, num_blocks, cache_stride_block,
                      cache_stride_token, cache_stride_head, block_tables, bt_stride, bt_width, query_start,
                      context_lens, nullptr, nullptr, nullptr, num_shares, nullptr, 0, 0, workspace, workspace_bytes,
                      out, out_stride_t, out_stride_h, num_heads, num_kv_heads, head_dim, block_size, scale, dtype,
                      stream, share_start, pieces);
}
