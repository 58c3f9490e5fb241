// Paged decode attention for gfx950: one query token per sequence, GQA.
//
// Replaces nimbus/kernels/paged_attention.py:25-146 (the Triton
// _paged_decode_kernel, _merge_partitions_kernel and their wrapper).
//
// The same kernels serve speculative verification (nimbus_paged_verify):
// every sequence then has nq query tokens, its newest nq positions, and
// query j sees keys 0 .. ctx - nq + j (the causal rule of
// nimbus/kernels/prefill_attention.py:27-78 for q_len = nq). The nq queries
// of a sequence become extra MFMA columns ("virtual heads": column = query j,
// head g), so each K/V page is read once for all of them.
//
// Work split (stream-K over the batch's pages). The 16-token pages of all
// sequences are laid end to end. For each kv-head group (a kv head and up to
// 16 of the query heads that share it, so each K/V page is read from HBM
// once) the launch has the same number of waves, and wave i takes the i-th
// equal slice of that page sequence. Every wave therefore streams the same
// number of bytes (+-1 page) whatever the mix of context lengths; a slice
// may end inside one sequence and continue into the next.
//
// The waves of the kv-head groups that read the same slice form one
// workgroup (up to 8 waves) and meet at a barrier every kSyncPages pages.
// Left to themselves the waves of different kv heads drift apart, and waves
// reading the same pages at different times slow each other down (measured:
// each kv head alone streams at one rate, but together some heads ended
// 25% later than others); kept in step, the heads of a page are read
// together and finish together. No atomics and no state are kept between
// calls. Wave 0 first turns context_lens into the page prefix sum in LDS;
// then every wave walks its kv group's slice one page at a time. Decode is
// bound by HBM latency as much as bandwidth, so each wave keeps kRing pages
// of K/V in flight in a ring of register buffers (page x + kRing is issued
// as soon as page x has been consumed), and finds each page's id kRing + 2
// pages ahead with scalar loads that never wait behind the vector loads.
// Per page, with the nq x G (query, head) columns padded to 16 per chunk:
//   S^T[token][g] = K[token][:] . Q^T[:][g]   (16x16x32 MFMA, K straight from
//                                               HBM into the A-operand layout)
//   online softmax per column g in fp32 (exp2 domain), reductions across the
//   four 16-lane groups with lane shuffles
//   O^T[d][g]    += V^T[d][token] . P^T[token][g]  (16x16x16 MFMA; P^T is
//                                               the QK output layout as is; V
//                                               is staged through LDS as
//                                               loaded and read back
//                                               transposed with
//                                               ds_read_b64_tr_b16)
// For bf16 the PV product keeps V exact and carries P as two bf16 terms
// (hi + lo, ~16 mantissa bits): rounding P to one bf16 alone costs ~8e-3
// at |o| ~ 0.5, beyond the output tolerance. For fp16, P is one fp16.
// When its slice covers a whole sequence the wave writes the normalised
// output. Otherwise it writes fp32 (O, m, l) for its piece to slot
// (wave + sequence), which no other wave uses, and paged_decode_merge_kernel
// combines the pieces (the reference's _merge_partitions_kernel rule).
//
// The grid depends only on host integers (batch, kv heads, max_context and
// the device's CU count), so a call is capturable in a hipGraph, and no
// workgroup is launched beyond what the chip holds at once.
#include <atomic>
#include <mutex>

#include "common.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

constexpr int kPage = 16;             // tokens per page (the only block size)
// Slices shorter than this only add merge work. Big batches never reach it
// (their slices are bounded by the resident waves); a short batch takes
// more, shorter slices: config 1 (16 sequences, 530 pages per kv
// head) measured 14.8 us per call at 8 pages, 12.7 at 4, 11.9 at 2, with
// configs 3 and 5 unchanged.
constexpr int kMinPagesPerWave = 2;
constexpr int kMaxDecodeBatch = 4096; // LDS holds the batch's page prefix sum
constexpr int kRegPrefixBatch = 64;   // up to this batch the prefix lives in registers, a lane per sequence
constexpr int kWavesPerCU = 8;        // two waves of the page kernel per SIMD
constexpr int kMaxWgWaves = 8;        // waves (kv-head groups) per workgroup
constexpr int kSyncPages = 4;         // pages between the workgroup's barriers
// Pages of K/V in flight per wave. Two, not three: measured in one process,
// alternating with a three-page ring on the same buffers, config 3 ran
// 1.0-1.2 us and config 5 0.2-0.6 us faster per call (bit-identical results,
// 204 registers against 236).
constexpr int kRing = 2;
constexpr int kMaxVerifyQueries = 16; // queries per sequence of a verify call
// Running-max floor: finite, below any score, so a column that sees no key
// in a piece (a verify query whose causal limit ends before the piece) keeps
// exp2(m - m) = 1 and weights exp2(-inf - m) = 0 instead of NaN.
constexpr float kNoScore = -1e30f;
// gfx950 parts have 256 CUs; launches never exceed this many resident waves,
// which keeps the workspace size a pure function of the call's shape.
constexpr int64_t kMaxResidentWaves = 256 * kWavesPerCU;

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
  int32_t* pre_out;  // workspace: the page prefix sum [B + 1], for the merge pass
  float* part_ml;    // workspace: [slot][nq * H][2] (m, l) of partial pieces
  float* part_o;     // workspace: [slot][nq * H][D] unnormalised O of partial pieces
  int32_t B, H, G, gchunks, kvg;
  int32_t nkv;       // kv heads
  int32_t nq;        // query tokens per sequence (1 for decode)
  int32_t nwk;       // waves launched per kv-head group (slices)
  int32_t wgw;       // waves per workgroup: kv groups sharing a slice, a divisor of kvg
  int32_t wgc;       // workgroups per slice: kvg / wgw
  int32_t max_ctx;   // context bound: min(max_context, block-table width * 16)
  float scale_log2;
};

__device__ __forceinline__ int clamp_page(int32_t pid, int32_t nb) {
  return static_cast<uint32_t>(pid) < static_cast<uint32_t>(nb) ? pid : 0;
}

__device__ __forceinline__ int pages_of(const DecodeArgs& a, int b) {
  const int ctx = min(a.ctx[b], a.max_ctx);
  return ctx > 0 ? (ctx + kPage - 1) / kPage : 0;
}

// p[i] for a wave-uniform i, read through the scalar cache: a load the
// kernel never writes, which therefore does not wait behind vector loads.
__device__ __forceinline__ int32_t scalar_load(const int32_t* p, int i) {
  typedef const __attribute__((address_space(4))) int32_t* const_ptr;
  return ((const_ptr)(p))[i];
}

// Waves per kv-head group that get a slice: all launched ones, unless the
// batch is so short that slices would drop below kMinPagesPerWave pages.
__device__ __forceinline__ int active_waves(int total_pages, int nwk) {
  return max(1, min(nwk, total_pages / kMinPagesPerWave));
}

// First page of slice i out of nw over total pages.
__device__ __forceinline__ int slice_start(int i, int nw, int total) {
  return static_cast<int>(static_cast<int64_t>(i) * total / nw);
}

// The slice holding page x: the largest i with slice_start(i) <= x.
__device__ __forceinline__ int slice_owner(int x, int nw, int total) {
  return static_cast<int>((static_cast<int64_t>(x + 1) * nw - 1) / total);
}

// Exclusive prefix sum of per-sequence page counts into pre[0..B], by the
// workgroup's first wave; every wave of the workgroup reads it after the
// barrier.
__device__ void page_prefix(const DecodeArgs& a, int* pre) {
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int per = (a.B + 63) / 64;
    const int lo = min(lane * per, a.B);
    const int hi = min(lo + per, a.B);
    int s = 0;
    for (int i = lo; i < hi; ++i) s += pages_of(a, i);
    int incl = s;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    int run = incl - s;
    for (int i = lo; i < hi; ++i) {
      pre[i] = run;
      run += pages_of(a, i);
    }
    if (lo < hi && hi == a.B) pre[a.B] = run;
  }
  __syncthreads();
}

// Slice and first kv group of workgroup w. The wgc workgroups of a slice
// sit 8 apart, so the dispatcher's round robin over the 8 XCDs puts them on
// one XCD (its L2 then serves a verify call's later column chunks, where
// they sit in other workgroups, the pages the first one fetched), and
// consecutive slices go to different XCDs.
__device__ __forceinline__ void wg_slice(const DecodeArgs& a, int w, int* idx, int* kg0) {
  const int C = a.wgc;
  const int full = (a.nwk / 8) * 8 * C;  // workgroups in whole groups of 8 slices
  int r, i;
  if (w < full) {
    const int rem = w % (8 * C);
    r = rem / 8;
    i = (w / (8 * C)) * 8 + rem % 8;
  } else {
    const int t = a.nwk % 8;
    const int rem = w - full;
    r = rem / t;
    i = (a.nwk / 8) * 8 + rem % t;
  }
  *idx = i;
  *kg0 = r * a.wgw;
}

template <int D>
struct PageBuf {
  static constexpr int KK = D / 32;           // 16x16x32 steps over the head dim
  static constexpr int VL = kPage * D / 512;  // 16-byte V loads per lane per page
  u32x4 k[KK];                                // K in the QK A-operand layout
  u32x4 v[VL];                                // V rows as loaded
};

// Where page p of sequence b lives (all wave-uniform). The loads are kept
// raw: what depends on them is computed where it is used, so nothing waits
// for them before it has to.
struct PageRef {
  int b, p, ctx_raw, pid_raw;
};

// Swizzled position of 16-byte chunk c of V row r in LDS: rows are read
// sixteen at a time by the transposed PV operand loads, and spreading equal
// chunks of different rows over different banks keeps those reads
// conflict-free up to the LDS bandwidth. At D = 64 two 128-byte rows share
// the 256 bytes the 64 banks serve per cycle (row parity picks the half), so
// the pattern uses row bits 1-2 there.
template <int D>
__device__ __forceinline__ int v_pos(int r, int c) {
  return D == 128 ? c ^ ((2 * r) & 15) : c ^ (r & 6);
}

// STREAM: K/V pages are loaded nontemporally (streamed, not kept in the L2).
// Every page is read once per launch when there is one column chunk, and
// streaming measured 5-6% faster there (config 3's page pass 86.6-88.0 us
// against 92.1-93.3); with two chunks the second chunk's reads of a page hit
// the L2 the first chunk filled, so those launches load ordinarily.
// STREAM: K/V pages loaded nontemporally (a launch with one column chunk
// reads every page once). REGP: the batch has at most kRegPrefixBatch
// sequences and its page prefix lives in registers (a compile-time choice:
// with both paths in one kernel the waits the LDS path needs are placed on
// the register path too).
template <int DT, int D, bool STREAM, bool REGP>
__global__ __launch_bounds__(64 * kMaxWgWaves) __attribute__((amdgpu_waves_per_eu(2))) void paged_decode_kernel(
    DecodeArgs a) {
  // (takes the kernel arguments the first page loads need, so that their
  // loads go out with the first ones instead of after the prefix, a round
  // trip of their own)
  asm volatile("" ::"s"(a.q), "s"(a.q_sb), "s"(a.q_sh), "s"(a.kc), "s"(a.vc), "s"(a.c_sb), "s"(a.c_st), "s"(a.c_sh),
               "s"(a.bt), "s"(a.bt_sb), "s"(a.num_blocks), "s"(a.ctx), "s"(a.B), "s"(a.nq), "s"(a.nwk), "s"(a.wgw),
               "s"(a.wgc), "s"(a.max_ctx));
  constexpr int KK = D / 32;
  constexpr int NN = D / 16;              // 16-row blocks of O^T
  constexpr int LPT = D / 8;              // lanes per token row (16 bytes each)
  constexpr int TPL = 64 / LPT;           // token rows per wave-wide load
  constexpr int VL = PageBuf<D>::VL;
  __shared__ __attribute__((aligned(16))) uint16_t vbs[kMaxWgWaves][kPage * D];  // per wave: a page of V, swizzled
  extern __shared__ int pre[];  // [B + 1]

  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int col = lane % 16;
  const int grp = lane / 16;
  uint16_t* const vb = vbs[wave];
  int idx, kg;
  wg_slice(a, blockIdx.x, &idx, &kg);
  // kv group kg is column chunk kg / nkv of kv head kg % nkv. With two
  // chunks and an even number of waves, a workgroup holds both chunks of
  // wgw / 2 kv heads (waves 2h and 2h + 1: chunks 0 and 1 of its h-th), so
  // the two waves that read a page walk it together on one CU and the
  // second finds it in the cache the first filled (measured 4% faster on
  // 16 x 5-token verify calls than a workgroup per chunk); otherwise the
  // workgroup's waves are consecutive kv groups.
  if (a.gchunks == 2 && (a.wgw & 1) == 0) kg = (wave & 1) * a.nkv + kg / 2 + (wave >> 1);
  else kg += wave;
  const int kvh = kg % a.nkv;
  const int g0 = (kg / a.nkv) * 16;
  const int vcol = g0 + col;  // virtual column: query vcol / G, head vcol % G
  const bool g_ok = vcol < a.nq * a.G;
  const int qj = g_ok ? vcol / a.G : 0;
  const int head = kvh * a.G + (g_ok ? vcol - qj * a.G : 0);
  const int back = a.nq - 1 - qj;  // keys this query sees fewer than the newest
  const int64_t vhead = static_cast<int64_t>(qj) * a.H + head;  // partial-piece row

  // The batch's page prefix. Up to 64 sequences (REGP) every wave holds it in
  // registers, lane i the pages of sequences 0..i (lanes past the batch:
  // INT32_MAX): a page's sequence is then a ballot, and neither LDS nor a
  // barrier stands between the context lengths and the page-id loads, which
  // all go out together. A larger batch keeps it in LDS (page_prefix), the
  // walk moving a cursor over it.
  constexpr bool reg_prefix = REGP;
  int incl = INT32_MAX;
  int total;
  if constexpr (reg_prefix) {
    int v = lane < a.B ? pages_of(a, lane) : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(v, off, 64);
      if (lane >= off) v += t;
    }
    if (lane < a.B) incl = v;
    total = __builtin_amdgcn_readlane(v, a.B - 1);  // (the host launches no empty batch)
    if (blockIdx.x == 0 && wave == 0) {
      if (lane == 0) a.pre_out[0] = 0;
      if (lane < a.B) a.pre_out[lane + 1] = v;
    }
  } else {
    page_prefix(a, pre);
    total = __builtin_amdgcn_readfirstlane(pre[a.B]);
    if (blockIdx.x == 0 && wave == 0) {
      for (int i = lane; i <= a.B; i += 64) a.pre_out[i] = pre[i];
    }
  }
  // Pages before sequence b (wave-uniform b <= B).
  auto prefix_at = [&](int b) {
    if constexpr (reg_prefix) return b == 0 ? 0 : __builtin_amdgcn_readlane(incl, b - 1);
    else return pre[b];
  };
  const int nw = active_waves(total, a.nwk);
  if (idx >= nw || total == 0) return;
  const int lo = slice_start(idx, nw, total);
  const int hi = slice_start(idx + 1, nw, total);
  if (lo >= hi) return;

  const uint16_t* kbase = a.kc + static_cast<int64_t>(kvh) * a.c_sh;
  const uint16_t* vbase = a.vc + static_cast<int64_t>(kvh) * a.c_sh;

  // Q^T as the B operand: column g, k-group grp holds q[g][32kk + 8grp .. +8].
  // Columns past nq x G read query 0, head kvh * G (a valid row) and are
  // never written, so the load needs no mask and nothing waits for it before
  // its first use.
  auto load_q = [&](int b, u32x4* dst) {
    const int64_t tok = static_cast<int64_t>(b) * a.nq + qj;
    const uint16_t* qrow = a.q + tok * a.q_sb + static_cast<int64_t>(head) * a.q_sh;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) dst[kk] = *reinterpret_cast<const u32x4*>(qrow + 32 * kk + 8 * grp);
  };

  // First sequence of the slice: the largest b with pre[b] <= lo; `cursor`
  // then only moves forward.
  int cursor = 0;
  if constexpr (!reg_prefix) {
    int l = 0, h = a.B;
    while (h - l > 1) {
      const int mid = (l + h) >> 1;
      if (pre[mid] <= lo) l = mid;
      else h = mid;
    }
    cursor = l;
  }
  // Sequence and page of flat page y < hi.
  auto place = [&](int y, PageRef& r) {
    if constexpr (reg_prefix) {
      // sequences that end at or before page y (y < total: at most B - 1)
      r.b = __builtin_popcountll(__builtin_amdgcn_ballot_w64(incl <= y));
      r.p = __builtin_amdgcn_readfirstlane(y - prefix_at(r.b));
    } else {
      while (pre[cursor + 1] <= y) ++cursor;
      r.b = __builtin_amdgcn_readfirstlane(cursor);
      r.p = __builtin_amdgcn_readfirstlane(y - pre[cursor]);
    }
  };
  auto locate = [&](int y) {
    PageRef r;
    if (y < hi) {
      place(y, r);
      r.ctx_raw = scalar_load(a.ctx, r.b);
      r.pid_raw = scalar_load(a.bt + r.b * a.bt_sb, r.p);
    } else {
      r.b = -1;
      r.p = 0;
      r.ctx_raw = 0;
      r.pid_raw = 0;
    }
    return r;
  };
  auto load_page = [&](PageBuf<D>& bf, const PageRef& r) {
    const int64_t off = static_cast<int64_t>(clamp_page(r.pid_raw, a.num_blocks)) * a.c_sb;
    // Rows of the page inside the context: the last page's rows past it are
    // not fetched (zeros; the softmax masks them anyway). Measured on one
    // process, alternating with the unmasked loads on the same buffers:
    // config 3 84.4-84.7 us per call against 84.8-85.2, config 5 +0.08%.
    const int vr = min(a.max_ctx, r.ctx_raw) - kPage * r.p;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u32x4* src = reinterpret_cast<const u32x4*>(kbase + off + col * a.c_st + 32 * kk + 8 * grp);
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (col < vr) {
        if constexpr (STREAM) v = __builtin_nontemporal_load(src);
        else v = *src;
      }
      bf.k[kk] = v;
    }
#pragma unroll
    for (int r2 = 0; r2 < VL; ++r2) {
      const int tt = r2 * TPL + lane / LPT;
      const u32x4* src = reinterpret_cast<const u32x4*>(vbase + off + tt * a.c_st + 8 * (lane % LPT));
      u32x4 v = u32x4{0u, 0u, 0u, 0u};
      if (tt < vr) {
        if constexpr (STREAM) v = __builtin_nontemporal_load(src);
        else v = *src;
      }
      bf.v[r2] = v;
    }
  };

  // ref[i] describes page x + i of the step about to run.
  PageRef ref[kRing + 2];
#pragma unroll
  for (int i = 0; i < kRing + 2; ++i) ref[i] = PageRef{-1, 0, 0, 0};
  {
    // The first kRing + 2 pages' table entries and context lengths: lane i
    // loads page lo + i's, two vector loads for all of them. As scalar loads
    // (what the walk uses, so that they never wait behind its K/V loads)
    // they took 3-12 us here on config 3's cold block tables, every wave of
    // the chip missing the scalar caches at once; no K/V load is in flight
    // yet for these to queue behind.
    int vb = 0, vp = 0;
    bool von = false;
#pragma unroll
    for (int i = 0; i < kRing + 2; ++i) {
      if (lo + i < hi) {
        place(lo + i, ref[i]);
        if (lane == i) {
          vb = ref[i].b;
          vp = ref[i].p;
          von = true;
        }
      }
    }
    const int vpid = von ? a.bt[static_cast<int64_t>(vb) * a.bt_sb + vp] : 0;
    const int vctx = von ? a.ctx[vb] : 0;
#pragma unroll
    for (int i = 0; i < kRing + 2; ++i) {
      if (lo + i < hi) {
        ref[i].pid_raw = __builtin_amdgcn_readlane(vpid, i);
        ref[i].ctx_raw = __builtin_amdgcn_readlane(vctx, i);
      }
    }
  }
  PageBuf<D> buf[kRing];
#pragma unroll
  for (int i = 0; i < kRing; ++i) {
    if (lo + i < hi) load_page(buf[i], ref[i]);
  }
  u32x4 qop[KK], qnext[KK];
  load_q(ref[0].b, qop);
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) qnext[kk] = qop[kk];

  // This lane's staging slots (row, swizzled chunk) and its transposed-read
  // addresses: lane j of group grp reads row 4 grp + j/4, elements
  // 16 nn + 4 (j%4) .. +4 (see lds_read_tr16).
  uint16_t* stage[VL];
#pragma unroll
  for (int r2 = 0; r2 < VL; ++r2) {
    const int tt = r2 * TPL + lane / LPT;
    stage[r2] = vb + tt * D + 8 * v_pos<D>(tt, lane % LPT);
  }
  const int tr_row = 4 * grp + col / 4;
  const uint16_t* tr_base = vb + tr_row * D + 4 * ((col % 4) % 2);
  const int tr_chunk = (col % 4) / 2;

  int seg0 = lo;  // first flat page of the current piece
  float m_run = kNoScore;
  float l_run = 0.f;
  f32x4 acc[NN];
#pragma unroll
  for (int nn = 0; nn < NN; ++nn) acc[nn] = f32x4{0.f, 0.f, 0.f, 0.f};

  // One page: consume buffer bf (page x), refill it with page x + kRing.
  auto step = [&](PageBuf<D>& bf, int x) {
    const PageRef cur = ref[0];
    const bool more = x + 1 < hi;
    const bool piece_ends = !more || ref[1].b != cur.b;
    ref[kRing + 1] = locate(x + kRing + 1);  // scalar loads, used two steps from now
    const int ctx_left = min(cur.ctx_raw, a.max_ctx) - kPage * cur.p;  // >= 1
    const int valid = min(kPage, ctx_left);

    // Stage V as loaded. Rows past the context (only on a sequence's last
    // page) are zeroed: P is 0 there, but 0 * garbage must not reach the sum.
    if (valid < kPage) {
#pragma unroll
      for (int r2 = 0; r2 < VL; ++r2) {
        if (r2 * TPL + lane / LPT >= valid) bf.v[r2] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int r2 = 0; r2 < VL; ++r2) *reinterpret_cast<u32x4*>(stage[r2]) = bf.v[r2];

    f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) s = mfma_16x16x32<DT>(bf.k[kk], qop[kk], s);

    // Refill this buffer (and fetch the next sequence's Q) before the
    // softmax and PV of this page.
    if (x + kRing < hi) load_page(bf, ref[kRing]);
    if (piece_ends && more) load_q(ref[1].b, qnext);

    // Causal limit of this column's query: rows below ctx_left - back.
    const int lim = ctx_left - back;
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float xs = 4 * grp + r < lim ? s[r] * a.scale_log2 : -INFINITY;
      s[r] = xs;
      mx = fmaxf(mx, xs);
    }
    mx = max_across_groups(mx);
    const float m_new = fmaxf(m_run, mx);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = fast_exp2(s[r] - m_new);
    l_run = l_run * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    // Once the running max settles it rarely moves: skip the rescale then.
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
      for (int nn = 0; nn < NN; ++nn) acc[nn] *= alpha;
    }

    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (DT == kBFloat16) {
      // V stays exact in bf16; P is carried as bf16 hi + lo (~16 bits).
      uint16_t hi16[4], lo16[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        hi16[r] = f32_to_bf16(p[r]);
        lo16[r] = f32_to_bf16(p[r] - bf16_to_f32(hi16[r]));
      }
      const u32x2 p_hi = u32x2{pack2(hi16[0], hi16[1]), pack2(hi16[2], hi16[3])};
      const u32x2 p_lo = u32x2{pack2(lo16[0], lo16[1]), pack2(lo16[2], lo16[3])};
#pragma unroll
      for (int nn = 0; nn < NN; ++nn) {
        const u32x2 vop = lds_read_tr16(tr_base + 8 * v_pos<D>(tr_row, 2 * nn + tr_chunk));
        acc[nn] = mfma_16x16x16<kBFloat16>(vop, p_hi, acc[nn]);
        acc[nn] = mfma_16x16x16<kBFloat16>(vop, p_lo, acc[nn]);
      }
    } else {
      const u32x2 pop = u32x2{pack2(f32_to_f16(p[0]), f32_to_f16(p[1])), pack2(f32_to_f16(p[2]), f32_to_f16(p[3]))};
#pragma unroll
      for (int nn = 0; nn < NN; ++nn) {
        const u32x2 vop = lds_read_tr16(tr_base + 8 * v_pos<D>(tr_row, 2 * nn + tr_chunk));
        acc[nn] = mfma_16x16x16<kFloat16>(vop, pop, acc[nn]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    if (piece_ends) {
      // Finish the piece [seg0, x] of sequence cur.b.
      const int rb = cur.b;
      const float l = sum_across_groups(l_run);
      const bool whole = seg0 == prefix_at(rb) && x + 1 == prefix_at(rb + 1);
      if (g_ok) {
        if (whole) {
          const float inv = l > 0.f ? 1.f / l : 0.f;  // a query that sees no key gives 0
          const int64_t tok = static_cast<int64_t>(rb) * a.nq + qj;
          uint16_t* orow = a.out + tok * a.o_sb + static_cast<int64_t>(head) * a.o_sh;
#pragma unroll
          for (int nn = 0; nn < NN; ++nn) {
            const f32x4 o = acc[nn];
            const u32x2 w = u32x2{pack2(Elem<DT>::from_f32(o[0] * inv), Elem<DT>::from_f32(o[1] * inv)),
                                  pack2(Elem<DT>::from_f32(o[2] * inv), Elem<DT>::from_f32(o[3] * inv))};
            *reinterpret_cast<u32x2*>(orow + 16 * nn + 4 * grp) = w;
          }
        } else {
          const int64_t row = (static_cast<int64_t>(idx) + rb) * a.nq * a.H + vhead;
          float* po = a.part_o + row * D;
#pragma unroll
          for (int nn = 0; nn < NN; ++nn) *reinterpret_cast<f32x4*>(po + 16 * nn + 4 * grp) = acc[nn];
          if (grp == 0) *reinterpret_cast<float2*>(a.part_ml + row * 2) = make_float2(m_run, l);
        }
      }
      m_run = kNoScore;
      l_run = 0.f;
#pragma unroll
      for (int nn = 0; nn < NN; ++nn) acc[nn] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) qop[kk] = qnext[kk];
      seg0 = x + 1;
    }
#pragma unroll
    for (int i = 0; i < kRing + 1; ++i) ref[i] = ref[i + 1];
    // Every wave of the workgroup has the same lo and hi: all reach each barrier.
    if ((x - lo) % kSyncPages == kSyncPages - 1) __builtin_amdgcn_s_barrier();
  };

  for (int x = lo; x < hi; x += kRing) {
#pragma unroll
    for (int k = 0; k < kRing; ++k) {
      if (x + k >= hi) break;
      step(buf[k], x + k);
    }
  }
}

// Second pass: for every sequence whose pages were split between waves,
// o = sum_i O_i w_i / sum_i L_i w_i with w_i = 2^(m_i - max m) over its
// pieces (nimbus/kernels/paged_attention.py:83-98). One workgroup per
// (sequence, kv-head group); sequences held whole by one wave exit at once.
// A lane owns one column of the group and 8 consecutive elements of d; the
// columns x D / 8 lanes this takes (64 for a decode kv head with G = 4) are
// repeated over the workgroup's 256 lanes as piece groups, and group j
// reads pieces i0 + j, i0 + j + groups, ..., kMergeBatch of them per round
// trip, every load of a batch issued before any is used. So a sequence's
// pieces (tens for a long context) arrive in one or two round trips; the
// groups' running (M, L, O) are then combined through LDS by the same rule.
constexpr int kMergeBatch = 8;
constexpr int kMergeThreads = 256;  // 16 columns x D / 8 lanes (D <= 128)

template <int DT, int D>
__global__ __launch_bounds__(kMergeThreads) void paged_decode_merge_kernel(DecodeArgs a) {
  constexpr int SEG = D / 8;  // lanes per column
  static_assert(16 * SEG <= kMergeThreads, "one lane per (column, 8 elements of d)");
  __shared__ float sm[kMergeThreads], sl[kMergeThreads];
  __shared__ f32x4 so[2][kMergeThreads];
  const int b = blockIdx.x;
  const int kg = blockIdx.y;
  const int total = a.pre_out[a.B];
  const int first = a.pre_out[b];
  const int last = a.pre_out[b + 1] - 1;
  if (total == 0 || last < first) return;
  const int nw = active_waves(total, a.nwk);
  const int i0 = slice_owner(first, nw, total);
  const int i1 = slice_owner(last, nw, total);
  if (i0 == i1) return;
  const int kvh = kg % a.nkv;
  const int g0 = (kg / a.nkv) * 16;
  const int gcount = min(16, a.nq * a.G - g0);
  const int lanes = gcount * SEG;            // lanes of one piece group
  const int groups = kMergeThreads / lanes;  // >= 1
  const int e = threadIdx.x;
  const int grp = e / lanes;
  const int el = e - grp * lanes;
  const int vcol = g0 + el / SEG;
  const int qj = vcol / a.G;
  const int head = kvh * a.G + vcol - qj * a.G;
  const int64_t vhead = static_cast<int64_t>(qj) * a.H + head;
  const int64_t cols = static_cast<int64_t>(a.nq) * a.H;  // rows per slot
  const int d0 = 8 * (el % SEG);

  float M = kNoScore, L = 0.f;
  f32x4 O0 = f32x4{0.f, 0.f, 0.f, 0.f}, O1 = O0;
  if (grp < groups) {
    for (int i = i0 + grp; i <= i1; i += groups * kMergeBatch) {
      float2 ml[kMergeBatch];
      f32x4 o0[kMergeBatch], o1[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        // Slots past the sequence's last piece are not loaded (a decode group
        // is one wave, so the branch is uniform there): with a few pieces per
        // sequence most of a batch's loads would otherwise fetch its last
        // piece again (config 3: 0.9 us per call, config 5 1.7 us).
        ml[u] = float2{kNoScore, 0.f};
        o0[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        o1[u] = o0[u];
        if (i + u * groups <= i1) {
          const int64_t row = (static_cast<int64_t>(i + u * groups) + b) * cols + vhead;
          ml[u] = *reinterpret_cast<const float2*>(a.part_ml + row * 2);
          o0[u] = *reinterpret_cast<const f32x4*>(a.part_o + row * D + d0);
          o1[u] = *reinterpret_cast<const f32x4*>(a.part_o + row * D + d0 + 4);
        }
      }
      float mx = M;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        if (i + u * groups <= i1) mx = fmaxf(mx, ml[u].x);
      }
      const float wo = fast_exp2(M - mx);
      L *= wo;
      O0 *= wo;
      O1 *= wo;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        if (i + u * groups <= i1) {
          const float wi = fast_exp2(ml[u].x - mx);
          L += ml[u].y * wi;
          O0 += o0[u] * wi;
          O1 += o1[u] * wi;
        }
      }
      M = mx;
    }
  }
  // Groups without pieces keep M = kNoScore, L = 0, O = 0 and weigh nothing
  // (group 0 always holds piece i0).
  sm[e] = M;
  sl[e] = L;
  so[0][e] = O0;
  so[1][e] = O1;
  __syncthreads();
  if (grp != 0) return;
  for (int g = 1; g < groups; ++g) M = fmaxf(M, sm[g * lanes + el]);
  const float w0 = fast_exp2(sm[el] - M);
  L *= w0;
  O0 *= w0;
  O1 *= w0;
  for (int g = 1; g < groups; ++g) {
    const int j = g * lanes + el;
    const float w = fast_exp2(sm[j] - M);
    L += sl[j] * w;
    O0 += so[0][j] * w;
    O1 += so[1][j] * w;
  }
  const float inv = L > 0.f ? 1.f / L : 0.f;
  const int64_t tok = static_cast<int64_t>(b) * a.nq + qj;
  uint16_t* orow = a.out + tok * a.o_sb + static_cast<int64_t>(head) * a.o_sh + d0;
  const u32x4 w = u32x4{pack2(Elem<DT>::from_f32(O0[0] * inv), Elem<DT>::from_f32(O0[1] * inv)),
                        pack2(Elem<DT>::from_f32(O0[2] * inv), Elem<DT>::from_f32(O0[3] * inv)),
                        pack2(Elem<DT>::from_f32(O1[0] * inv), Elem<DT>::from_f32(O1[1] * inv)),
                        pack2(Elem<DT>::from_f32(O1[2] * inv), Elem<DT>::from_f32(O1[3] * inv))};
  *reinterpret_cast<u32x4*>(orow) = w;
}

// Waves the launch gives each kv-head group: what the chip keeps resident,
// capped by the pages the batch can hold (at least one).
static int64_t waves_per_group(int64_t cus, int kvg, int64_t max_pages) {
  const int64_t resident = cus * kWavesPerCU < kMaxResidentWaves ? cus * kWavesPerCU : kMaxResidentWaves;
  int64_t n = resident / kvg;
  if (n > max_pages / kMinPagesPerWave) n = max_pages / kMinPagesPerWave;
  return n < 1 ? 1 : n;
}

// CU count of the current device, asked of the runtime once per device and
// kept (a device's CU count does not change while the process runs).
constexpr int kMaxDevices = 64;
static std::atomic<int> g_device_cus[kMaxDevices];  // 0: not asked yet

int device_cus(int64_t* cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  const bool slot = dev >= 0 && dev < kMaxDevices;
  int n = slot ? g_device_cus[dev].load(std::memory_order_relaxed) : 0;
  if (n <= 0) {
    e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return static_cast<int>(e);
    if (slot) g_device_cus[dev].store(n, std::memory_order_relaxed);
  }
  *cus = n;
  return 0;
}

// phase bit 1: page pass, bit 2: merge pass.
template <int DT, int D>
static int launch_decode(const DecodeArgs& a, int phases, hipStream_t stream) {
  if (phases & 1) {
    const size_t dyn = static_cast<size_t>(a.B + 1) * sizeof(int);
    const dim3 grid(a.nwk * a.wgc), block(64 * a.wgw);
    const bool regp = a.B <= kRegPrefixBatch;
    if (a.gchunks == 1) {
      if (regp) hipLaunchKernelGGL((paged_decode_kernel<DT, D, true, true>), grid, block, dyn, stream, a);
      else hipLaunchKernelGGL((paged_decode_kernel<DT, D, true, false>), grid, block, dyn, stream, a);
    } else {
      if (regp) hipLaunchKernelGGL((paged_decode_kernel<DT, D, false, true>), grid, block, dyn, stream, a);
      else hipLaunchKernelGGL((paged_decode_kernel<DT, D, false, false>), grid, block, dyn, stream, a);
    }
  }
  if (phases & 2) {
    hipLaunchKernelGGL((paged_decode_merge_kernel<DT, D>), dim3(a.B, a.kvg), dim3(kMergeThreads), 0, stream, a);
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace nimbus

using namespace nimbus;

// Workspace layout, each part 256-byte aligned: page prefix [B + 1] int32;
// per slot (wave index + sequence, < waves per kv group + B) and (query,
// head) column the (m, l) pair; per slot and column D floats of O.
static int64_t round256(int64_t n) { return (n + 255) / 256 * 256; }
static int64_t prefix_bytes(int64_t batch) { return round256((batch + 1) * 4); }

static int64_t max_pages_of(int64_t batch, int64_t max_context) {
  return batch * ((max_context + kPage - 1) / kPage);
}

static int64_t workspace_size(int32_t batch, int32_t num_heads, int32_t head_dim, int64_t max_context,
                              int32_t nq) {
  if (batch < 0 || num_heads <= 0 || head_dim <= 0 || max_context < 0 || nq <= 0) return -1;
  // Any device and any kvg >= 1 launch at most this many waves per kv group.
  const int64_t slots = waves_per_group(kMaxResidentWaves, 1, max_pages_of(batch, max_context)) + batch;
  const int64_t cols = static_cast<int64_t>(num_heads) * nq;
  return prefix_bytes(batch) + round256(slots * cols * 2 * 4) + slots * cols * head_dim * 4;
}

extern "C" int64_t nimbus_paged_decode_workspace_bytes(int32_t batch, int32_t num_heads, int32_t head_dim,
                                                       int64_t max_context) {
  return workspace_size(batch, num_heads, head_dim, max_context, 1);
}

extern "C" int64_t nimbus_paged_verify_workspace_bytes(int32_t batch, int32_t queries_per_seq, int32_t num_heads,
                                                       int32_t head_dim, int64_t max_context) {
  if (queries_per_seq > kMaxVerifyQueries) return -1;
  return workspace_size(batch, num_heads, head_dim, max_context, queries_per_seq);
}

static int paged_decode_impl(int phases, int32_t nq, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* k_cache,
                             const void* v_cache, int64_t num_blocks, int64_t cache_stride_block,
                             int64_t cache_stride_token, int64_t cache_stride_head, const int32_t* block_tables,
                             int64_t bt_stride, int32_t bt_width, const int32_t* context_lens, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                             int32_t batch, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                             int32_t block_size, int64_t max_context, float scale, int32_t dtype, void* stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return NIMBUS_ERR_INVALID;
  if (nq <= 0) return NIMBUS_ERR_INVALID;
  if (nq > kMaxVerifyQueries) return NIMBUS_ERR_UNSUPPORTED;
  // Pages of other than 16 tokens and head dims other than 64 and 128 take
  // the general kernel (paged_general.hip).
  const bool general = general_shape(head_dim, block_size);
  if (general) {
    const int rc = general_check(head_dim, block_size);
    if (rc != 0) return rc;
  }
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (batch > kMaxDecodeBatch || max_context > (int64_t{1} << 30)) return NIMBUS_ERR_UNSUPPORTED;
  if (batch == 0 || max_context <= 0) return NIMBUS_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out) return NIMBUS_ERR_INVALID;
  if (num_blocks <= 0 || num_blocks > INT32_MAX || bt_width <= 0) return NIMBUS_ERR_INVALID;
  if (general) {
    // (element loads: no alignment asked of the strides; no workspace used)
    if (phases != 3) return NIMBUS_ERR_UNSUPPORTED;  // one launch: there are no pieces to merge
    AttnGeneralArgs g{};
    g.q = static_cast<const uint16_t*>(q);
    g.q_st = q_stride_b;
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
    g.nq = nq;
    g.max_ctx = static_cast<int32_t>(max_context);
    g.out = static_cast<uint16_t*>(out);
    g.o_st = out_stride_b;
    g.o_sh = out_stride_h;
    g.H = num_heads;
    g.G = num_heads / num_kv_heads;
    g.KV = num_kv_heads;
    g.D = head_dim;
    g.scale_log2 = scale * 1.4426950408889634f;
    if (static_cast<int64_t>(bt_width) * block_size > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
    return launch_general_decode(g, batch, dtype, static_cast<hipStream_t>(stream));
  }
  // 16-byte vector access: 8-element aligned strides and bases.
  if ((q_stride_b | q_stride_h | cache_stride_block | cache_stride_token | cache_stride_head | out_stride_b |
       out_stride_h) % 8 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
       reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(workspace)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  const int64_t need = workspace_size(batch, num_heads, head_dim, max_context, nq);
  if (need < 0) return NIMBUS_ERR_INVALID;
  if (workspace == nullptr || workspace_bytes < need) return NIMBUS_ERR_WORKSPACE;
  int64_t cus = 0;
  const int rc = device_cus(&cus);
  if (rc != 0) return rc;

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
  a.B = batch;
  a.H = num_heads;
  a.G = num_heads / num_kv_heads;
  a.nq = nq;
  a.nkv = num_kv_heads;
  a.gchunks = (nq * a.G + 15) / 16;
  a.kvg = num_kv_heads * a.gchunks;
  const int64_t ctx_bound = max_context < static_cast<int64_t>(bt_width) * kPage
                                ? max_context
                                : static_cast<int64_t>(bt_width) * kPage;
  a.max_ctx = static_cast<int32_t>(ctx_bound);
  // Never more waves per group than the workspace's slots were sized for.
  const int64_t nwk = waves_per_group(cus, a.kvg, max_pages_of(batch, ctx_bound));
  a.nwk = static_cast<int32_t>(nwk);
  // Kv groups share a workgroup when the launch fills the chip; a shorter
  // batch keeps one-wave workgroups, spread over every CU.
  a.wgw = 1;
  const int64_t resident = cus * kWavesPerCU < kMaxResidentWaves ? cus * kWavesPerCU : kMaxResidentWaves;
  const bool fills = (nwk + 1) * a.kvg > resident;  // one more wave per group would not fit
  for (int w = kMaxWgWaves; w > 1 && fills; --w) {
    if (a.kvg % w == 0) {
      a.wgw = w;
      break;
    }
  }
  a.wgc = a.kvg / a.wgw;
  if (nwk * a.kvg > INT32_MAX / 2 || max_pages_of(batch, ctx_bound) > INT32_MAX / 2) return NIMBUS_ERR_UNSUPPORTED;
  const int64_t slots = nwk + batch;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  a.pre_out = reinterpret_cast<int32_t*>(ws);
  a.part_ml = reinterpret_cast<float*>(ws + prefix_bytes(batch));
  const int64_t cols = static_cast<int64_t>(num_heads) * nq;
  a.part_o = reinterpret_cast<float*>(ws + prefix_bytes(batch) + round256(slots * cols * 2 * 4));
  a.scale_log2 = scale * 1.4426950408889634f;

  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == kFloat16) {
    return head_dim == 64 ? launch_decode<kFloat16, 64>(a, phases, s) : launch_decode<kFloat16, 128>(a, phases, s);
  }
  return head_dim == 64 ? launch_decode<kBFloat16, 64>(a, phases, s) : launch_decode<kBFloat16, 128>(a, phases, s);
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

extern "C" int nimbus_paged_decode(NIMBUS_DECODE_PARAMS) { return paged_decode_impl(3, 1, NIMBUS_DECODE_ARGS); }

extern "C" int nimbus_paged_decode_pages(NIMBUS_DECODE_PARAMS) {
  return paged_decode_impl(1, 1, NIMBUS_DECODE_ARGS);
}

extern "C" int nimbus_paged_decode_merge(NIMBUS_DECODE_PARAMS) {
  return paged_decode_impl(2, 1, NIMBUS_DECODE_ARGS);
}

// ---------------------------------------------------------------- allocation-free decode
//
// nimbus_paged_decode_noalloc runs nimbus_paged_decode's kernels with their
// workspace in `scratch`, a file-scope device array of kNoAllocScratchBytes:
// each device the library runs on holds its own copy until the process
// ends, and every call on that device shares it. In host code `scratch`
// names a host-side stand-in, not device memory: the device address comes
// from hipGetSymbolAddress, asked once per device (with that device
// current) on the entry point's first call there, and only that address is
// handed to kernels. The decode workspace needs no initialisation (the page
// pass writes the prefix sum and every piece before the merge reads them),
// so nothing is cleared. Calls that overlap on one device race on it.
constexpr int64_t kNoAllocScratchBytes = NIMBUS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

static std::atomic<void*> g_scratch_addr[kMaxDevices];  // null: not asked yet
static std::mutex g_scratch_mu;

// Device address of the current device's `scratch`.
static int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return NIMBUS_ERR_UNSUPPORTED;
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

extern "C" int nimbus_paged_decode_noalloc(const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                           const void* k_cache, const void* v_cache, int64_t num_blocks,
                                           int64_t cache_stride_block, int64_t cache_stride_token,
                                           int64_t cache_stride_head, const int32_t* block_tables, int64_t bt_stride,
                                           int32_t bt_width, const int32_t* context_lens, void* out,
                                           int64_t out_stride_b, int64_t out_stride_h, int32_t batch,
                                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                           int32_t block_size, int64_t max_context, float scale, int32_t dtype,
                                           void* stream) {
  const int64_t need = workspace_size(batch, num_heads, head_dim, max_context, 1);
  if (need < 0) return NIMBUS_ERR_INVALID;
  if (need > kNoAllocScratchBytes) return NIMBUS_ERR_SCRATCH;
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != 0) return rc;
  return paged_decode_impl(3, 1, q, q_stride_b, q_stride_h, k_cache, v_cache, num_blocks, cache_stride_block,
                           cache_stride_token, cache_stride_head, block_tables, bt_stride, bt_width, context_lens,
                           out, out_stride_b, out_stride_h, ws, kNoAllocScratchBytes, batch, num_heads, num_kv_heads,
                           head_dim, block_size, max_context, scale, dtype, stream);
}

// q and out hold batch * queries_per_seq tokens in sequence order (token
// b * queries_per_seq + j is query j of sequence b); the stride arguments
// named _b are per token.
extern "C" int nimbus_paged_verify(int32_t queries_per_seq, NIMBUS_DECODE_PARAMS) {
  return paged_decode_impl(3, queries_per_seq, NIMBUS_DECODE_ARGS);
}
