// INT8 weight-only matmul for gfx950: y = dtype(fp32(x @ w_q^T) * scale).
//
// Replaces nimbus/kernels/int8_matmul.py:26-64 (the Triton
// _int8_matmul_kernel and its wrapper), which Int8Linear
// (nimbus/quant/int8.py:32-47) runs for the decoder projections. x is fp16
// or bf16 [M, K]; w_q int8 [N, K] (round(w / scale), |w_q| <= 127, per
// output channel); scale [N] in x's dtype; y [M, N] in x's dtype.
//
// Decode is bound by reading the weights, so every weight byte is streamed
// from HBM once per launch:
// - a workgroup of 8 waves owns 128 output channels, 16 per wave (the rows
//   of a 16x16x32 MFMA's A operand), over one range of K;
// - each lane loads 16 consecutive int8 of its row per 64-k step, kRing
//   steps ahead, and converts them exactly to fp16 / bf16 in registers
//   (|w_q| <= 127 fits either type's significand);
// - x's 64-k step for the workgroup's tokens is staged in LDS once and read
//   by all 8 waves; its global loads ride the same kRing-deep register ring
//   as the weights, so waiting for one never drains the other (the
//   tile-order kernel further down loads x straight into LDS instead);
// - the k order inside a step is the same permutation for both operands, so
//   one 16-byte weight load feeds two MFMAs: chunk 0 takes k = 16g + 0..7 of
//   lane group g, chunk 1 takes k = 16g + 8..15 (the sum over k does not
//   depend on the order).
// When the output channels alone would leave CUs idle, K is split between
// workgroups: each writes its fp32 partial sums, and
// int8_matmul_reduce_kernel adds them in split order (the result does not
// depend on timing), scales and rounds.
#include <type_traits>

#include "common.h"
#include "nimbus_attn_internal.h"
#include "int8_epilogue.h"
#include "silu.h"

namespace nimbus {

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kGemmRows = 16 * kGemmWaves;  // output channels per workgroup
constexpr int kGemmStep = 64;               // k per pipeline step
constexpr int kGemmRing = 8;                // steps of loads in flight
// One token's step of x in LDS: 128 bytes, eight 16-byte chunks in swizzled
// order (x_chunk).
constexpr int kXRow = 2 * kGemmStep;
constexpr int kMaxSplits = 16;
constexpr int kMinSplitK = kGemmRing * kGemmStep;  // splits are whole rings of steps
constexpr int kFillWorkgroups = 256;        // one per CU of a gfx950 part

constexpr uint32_t kOutOfRange = 0xFFFFFFF0u;     // a buffer offset past any operand: reads zero

struct GemmArgs {
  const uint16_t* x;
  int32_t sx;        // elements; x spans x_bytes < 2^31
  const int8_t* w;
  int32_t sw;        // bytes; w spans w_bytes < 2^31
  int32_t x_bytes, w_bytes;
  const uint16_t* scale;
  uint16_t* y;
  int64_t sy;
  float* part;  // [splits][M][N] fp32 partial sums (splits > 1)
  int32_t M, N, K;
  int32_t splits, ksplit;  // ksplit: k per split, a multiple of kMinSplitK
};

typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

// LDS position of 16-byte chunk c (k = 8 c .. 8 c + 7 of the step) in the row
// of token t. Lane group g reads chunks 2 g and 2 g + 1 (its two MFMA
// operands) of sixteen consecutive tokens; those land in physical chunks g
// and g + 4, XOR-ed with the token's low three bits. With padded rows (144
// bytes, chunks in order) the counters read bank conflicts in 39-44% of the
// LDS's active cycles; with this order, none.
__device__ __forceinline__ int x_chunk(int t, int c) {
  return ((c >> 1) | ((c & 1) << 2)) ^ (t & 7);
}

// x_chunk's inverse: the chunk stored at position p of token t's row.
__device__ __forceinline__ int x_chunk_at(int t, int p) {
  const int u = p ^ (t & 7);
  return ((u << 1) & 6) | (u >> 2);
}

// Eight int8 (two dwords) -> the eight fp16 / bf16 of an MFMA operand.
template <int DT>
__device__ __forceinline__ u32x4 i8x8_to_operand(uint32_t w0, uint32_t w1);

// fp16: byte b + 128 goes under the exponent of 1024 (0x64XX is 1024 + XX)
// and 1152 is subtracted; both steps are exact.
__device__ __forceinline__ u32x2 i8x4_to_f16x4(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [1024 + u0, 1024 + u1]
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [1024 + u2, 1024 + u3]
  const h16x2 bias = h16x2{static_cast<_Float16>(-1152.f), static_cast<_Float16>(-1152.f)};
  return u32x2{__builtin_bit_cast(uint32_t, __builtin_bit_cast(h16x2, lo) + bias),
               __builtin_bit_cast(uint32_t, __builtin_bit_cast(h16x2, hi) + bias)};
}

template <>
__device__ __forceinline__ u32x4 i8x8_to_operand<kFloat16>(uint32_t w0, uint32_t w1) {
  const u32x2 a = i8x4_to_f16x4(w0), b = i8x4_to_f16x4(w1);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// bf16: each byte, sign-extended, converts to fp32 exactly (one
// v_cvt_f32_i32 whose SDWA operand select picks and extends the byte), and
// the upper half of that fp32 is the byte's bf16, exactly (|b| <= 128 needs
// at most 8 significant bits). Six VALU ops per four weights.
// (The byte is moved to the top in unsigned arithmetic, then shifted back
// down arithmetically: a left shift of a negative int32 is undefined.)
__device__ __forceinline__ u32x2 i8x4_to_bf16x4(uint32_t w) {
  const float f0 = static_cast<float>(static_cast<int32_t>(w << 24) >> 24);
  const float f1 = static_cast<float>(static_cast<int32_t>(w << 16) >> 24);
  const float f2 = static_cast<float>(static_cast<int32_t>(w << 8) >> 24);
  const float f3 = static_cast<float>(static_cast<int32_t>(w) >> 24);
  // upper halves of (f0, f1) and (f2, f3)
  return u32x2{__builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u),
               __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u)};
}

template <>
__device__ __forceinline__ u32x4 i8x8_to_operand<kBFloat16>(uint32_t w0, uint32_t w1) {
  const u32x2 a = i8x4_to_bf16x4(w0), b = i8x4_to_bf16x4(w1);
  return u32x4{a[0], a[1], b[0], b[1]};
}

// Workgroup barrier that waits only for LDS traffic, so the weight loads in
// flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Waits until at most N of this wave's vector-memory loads are outstanding
// (gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at
// their maxima, i.e. not waited for). Loads return in issue order, so every
// load issued before the last N has landed.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt holds six bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane from a buffer straight into LDS: lane l's land at
// lds + 16 l (lds is the same for the whole wave). A non-template function,
// so that the host pass, which cannot form the LDS pointer, only defers its
// complaint about this body instead of dropping the kernels' host stubs.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, off, 0, 0, 0);
}

// Workgroup barrier for x loaded straight into LDS: each wave first waits
// until its loads older than the last N have written LDS, so after the
// barrier every wave's part of those steps is there. The compiler does not
// count these loads against later LDS reads of the same array, and the
// workgroup fence would wait for every load in flight (the weight ring
// too), hence the count by hand; the signal fences keep the compiler from
// moving LDS accesses across the barrier.
template <int N>
__device__ __forceinline__ void dma_barrier() {
  wait_vm<N>();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Grid: (N / 128 channel tiles, splits, M / BM token tiles).
template <int DT, int BM>
__global__ __launch_bounds__(kGemmThreads) void int8_matmul_kernel(GemmArgs a) {
  constexpr int CB = BM / 16;   // 16-token column blocks
  constexpr int XT = BM * 8;    // threads staging x: one 16-byte chunk of a token's step each
  static_assert(XT <= kGemmThreads, "x staging needs one thread per chunk");
  __shared__ __attribute__((aligned(16))) uint8_t xs[2][BM * kXRow];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  const int col = lane % 16;
  const int grp = lane / 16;
  const int n0 = blockIdx.x * kGemmRows + 16 * wave;
  const int kb = blockIdx.y * a.ksplit;
  const int ke = min(a.K, kb + a.ksplit);
  const int m0 = blockIdx.z * BM;
  const int steps = (ke - kb + kGemmStep - 1) / kGemmStep;

  // Loads are unconditional buffer loads: a masked lane's offset is past the
  // buffer's end and reads zeros, so no branch (and no full wait for the
  // loads in flight) is needed to skip it.
  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(a.w), 0, __builtin_amdgcn_readfirstlane(a.w_bytes), kBufferFlags);
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), 0, __builtin_amdgcn_readfirstlane(a.x_bytes), kBufferFlags);
  // This lane's weight row (rows past N read row N - 1 and are never stored).
  const uint32_t woff = static_cast<uint32_t>(min(n0 + col, a.N - 1) * a.sw + kb + 16 * grp);
  auto load_w = [&](int s) {
    const bool on = kb + kGemmStep * s + 16 * grp < ke;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         wrsrc, on ? woff + kGemmStep * s : kOutOfRange, 0, 0));
  };
  // x staging: thread t < XT moves token t / 8, 16-byte chunk t % 8 of each
  // step; tokens past M and k past the range stage zeros.
  const int xt_tok = tid / 8;
  const int xt_chunk = tid % 8;
  const bool xt_on = tid < XT && m0 + xt_tok < a.M;
  const uint32_t xoff = xt_on ? static_cast<uint32_t>(2 * ((m0 + xt_tok) * a.sx + kb + 8 * xt_chunk)) : 0u;
  auto load_x = [&](int s) {
    const bool on = xt_on && kb + kGemmStep * s + 8 * xt_chunk < ke;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         xrsrc, on ? xoff + 2 * kGemmStep * s : kOutOfRange, 0, 0));
  };
  const int xs_off = xt_tok * kXRow + 16 * x_chunk(xt_tok, xt_chunk);

  u32x4 wr[kGemmRing], xr[kGemmRing];
#pragma unroll
  for (int j = 0; j < kGemmRing; ++j) {
    wr[j] = load_w(j);
    xr[j] = load_x(j);
  }
  if (tid < XT) *reinterpret_cast<u32x4*>(&xs[0][xs_off]) = xr[0];
  lds_barrier();

  f32x4 acc[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int xb_off = col * kXRow;  // B operand: token col of a block (its chunks 2 grp, 2 grp + 1)
  const int xc0 = 16 * x_chunk(col, 2 * grp), xc1 = 16 * x_chunk(col, 2 * grp + 1);

  // Whole rings of steps: a step past the range loads zeros (out-of-range
  // offsets) for both operands and adds exactly 0, and the ring's registers
  // keep their places across iterations (no copies that would wait for
  // loads in flight).
  for (int s0 = 0; s0 < steps; s0 += kGemmRing) {
#pragma unroll
    for (int j = 0; j < kGemmRing; ++j) {
      const int s = s0 + j;
      const uint8_t* xb = &xs[s & 1][xb_off];
      const u32x4 wv = wr[j];
      const u32x4 a0 = i8x8_to_operand<DT>(wv[0], wv[1]);
      const u32x4 a1 = i8x8_to_operand<DT>(wv[2], wv[3]);
      // Refill this ring slot: x(s) left it for LDS at the end of step s - 1.
      wr[j] = load_w(s + kGemmRing);
      xr[j] = load_x(s + kGemmRing);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(xb + cb * 16 * kXRow + xc0);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(xb + cb * 16 * kXRow + xc1);
        acc[cb] = mfma_16x16x32<DT>(a0, b0, acc[cb]);
        acc[cb] = mfma_16x16x32<DT>(a1, b1, acc[cb]);
      }
      // Stage x(s + 1) in the other buffer: every wave finished reading it
      // (step s - 1) before the last barrier.
      if (tid < XT) *reinterpret_cast<u32x4*>(&xs[(s + 1) & 1][xs_off]) = xr[(j + 1) % kGemmRing];
      lds_barrier();
    }
  }

  // Lane (col, grp) holds token m0 + 16 cb + col, channels n0 + 4 grp + r.
  const int n = n0 + 4 * grp;
  if (n >= a.N) return;
  if (a.splits == 1) {
    const u32x2 sw = *reinterpret_cast<const u32x2*>(a.scale + n);
    const float sc[4] = {Elem<DT>::to_f32(static_cast<uint16_t>(sw[0])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[0] >> 16)),
                         Elem<DT>::to_f32(static_cast<uint16_t>(sw[1])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[1] >> 16))};
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int m = m0 + 16 * cb + col;
      if (m < a.M) {
        const f32x4 o = acc[cb];
        const u32x2 v = u32x2{pack2(scaled<DT>(o[0], sc[0]), scaled<DT>(o[1], sc[1])),
                              pack2(scaled<DT>(o[2], sc[2]), scaled<DT>(o[3], sc[3]))};
        *reinterpret_cast<u32x2*>(a.y + static_cast<int64_t>(m) * a.sy + n) = v;
      }
    }
  } else {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int m = m0 + 16 * cb + col;
      if (m < a.M) {
        float* p = a.part + (static_cast<int64_t>(blockIdx.y) * a.M + m) * a.N + n;
        *reinterpret_cast<f32x4*>(p) = acc[cb];
      }
    }
  }
}

// Sum of the split partials in split order, scaled and rounded: one thread
// per 4 consecutive outputs of a row.
template <int DT>
__global__ __launch_bounds__(256) void int8_matmul_reduce_kernel(GemmArgs a) {
  const int64_t quads = static_cast<int64_t>(a.M) * (a.N / 4);
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= quads) return;
  const int m = static_cast<int>(i / (a.N / 4));
  const int n = static_cast<int>(i % (a.N / 4)) * 4;
  const int64_t plane = static_cast<int64_t>(a.M) * a.N;
  const float* p = a.part + static_cast<int64_t>(m) * a.N + n;
  f32x4 s = *reinterpret_cast<const f32x4*>(p);
  for (int k = 1; k < a.splits; ++k) s += *reinterpret_cast<const f32x4*>(p + k * plane);
  const u32x2 sw = *reinterpret_cast<const u32x2*>(a.scale + n);
  const float sc[4] = {Elem<DT>::to_f32(static_cast<uint16_t>(sw[0])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[0] >> 16)),
                       Elem<DT>::to_f32(static_cast<uint16_t>(sw[1])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[1] >> 16))};
  const u32x2 v = u32x2{pack2(scaled<DT>(s[0], sc[0]), scaled<DT>(s[1], sc[1])),
                        pack2(scaled<DT>(s[2], sc[2]), scaled<DT>(s[3], sc[3]))};
  *reinterpret_cast<u32x2*>(a.y + static_cast<int64_t>(m) * a.sy + n) = v;
}

// Tokens per workgroup tile for M tokens.
static int gemm_bm(int64_t m) { return m <= 16 ? 16 : (m <= 32 ? 32 : 64); }

// K split: enough workgroups to give every CU one, each split a whole number
// of rings of steps. A pure function of the shape.
static void gemm_split(int64_t m, int32_t n, int32_t k, int32_t* splits, int32_t* ksplit) {
  const int64_t tiles = ((n + kGemmRows - 1) / kGemmRows) * ((m + gemm_bm(m) - 1) / gemm_bm(m));
  int64_t s = 1;
  if (tiles < kFillWorkgroups) s = (kFillWorkgroups + tiles - 1) / tiles;
  if (s > kMaxSplits) s = kMaxSplits;
  if (s > k / kMinSplitK) s = k / kMinSplitK;
  if (s < 1) s = 1;
  int64_t ks = (k + s - 1) / s;
  ks = (ks + kMinSplitK - 1) / kMinSplitK * kMinSplitK;
  *ksplit = static_cast<int32_t>(ks);
  *splits = static_cast<int32_t>((k + ks - 1) / ks);
}

template <int DT, int BM>
static int launch_gemm(const GemmArgs& a, hipStream_t s) {
  const dim3 grid((a.N + kGemmRows - 1) / kGemmRows, a.splits, (a.M + BM - 1) / BM);
  hipLaunchKernelGGL((int8_matmul_kernel<DT, BM>), grid, dim3(kGemmThreads), 0, s, a);
  if (a.splits > 1) {
    const int64_t quads = static_cast<int64_t>(a.M) * (a.N / 4);
    hipLaunchKernelGGL((int8_matmul_reduce_kernel<DT>), dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256),
                       0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

template <int DT>
static int launch_gemm_dt(const GemmArgs& a, hipStream_t s) {
  switch (gemm_bm(a.M)) {
    case 16: return launch_gemm<DT, 16>(a, s);
    case 32: return launch_gemm<DT, 32>(a, s);
    default: return launch_gemm<DT, 64>(a, s);
  }
}

// ---------------------------------------------------------------- packed weights
//
// nimbus_int8_matmul_packed takes the weights in MFMA tile order (built once
// by nimbus_int8_pack_weight when a layer is quantized): block (nb, kc) of
// [ceil(N/16)][ceil(K/64)] is 1024 bytes, lane l's 16 at offset 16 l holding
// row 16 nb + l % 16, k = 64 kc + 16 (l / 16) .. +16 (zero padded), i.e.
// exactly the A operand one 16-byte load per lane feeds. A wave's weight
// loads are therefore 1 KB contiguous, and a wave streams one contiguous run
// of 16 K bytes. The 8 waves of a workgroup are RB row-block groups x KS k
// slices (RB x KS = 8, BM x KS <= 128); a wave computes RW row blocks (1 or
// 2) from each x operand it reads. Waves of one group take interleaved 64-k
// chunks and their sums are added in LDS at the end (fixed order), so narrow
// matrices need no cross-workgroup split for small M. x goes from memory
// straight into LDS (buffer loads with the LDS bit: no registers, no LDS
// write instructions), kXLead steps ahead into a ring of kXBufs buffers. A
// step reads all of its x operands from LDS at once and runs its MFMAs on
// weights converted during the previous step, converting the next step's
// weights while they execute; the workgroup meets at a barrier every second
// step.

constexpr int kPackRing = 4;  // steps of weight loads in flight
constexpr int kXBufs = 8;     // x steps in LDS
constexpr int kXLead = kXBufs - 2;  // x loaded this many steps ahead

template <int BM, int KS, int RW>
struct PackShape {
  static constexpr int RB = kGemmWaves / KS;                 // row-block groups per workgroup
  static constexpr int XP = BM * KS * 8;                     // 16-byte x pieces per step
  static constexpr int XC = (XP + kGemmThreads - 1) / kGemmThreads;  // pieces a thread stages per step
};

// Grid: (ceil(N / 16 / (RB RW)) row tiles, splits, M / BM token tiles).
// SILU: the projection is Llama's gate_up (gate rows [0, N/2), up rows
// [N/2, N)) and y = silu(gate) * up, [M, N/2]: the first RB/2 row-block groups
// of a workgroup take gate rows and the others the matching up rows, so that
// after the k-slice sum each up wave hands its rounded outputs to its gate
// partner through LDS (one split only; grid x = ceil(N / 32 / (RB/2 RW))).
template <int DT, int BM, int KS, int RW, bool SILU>
__global__ __launch_bounds__(kGemmThreads) void int8_matmul_packed_kernel(GemmArgs a) {
  constexpr int CB = BM / 16;
  constexpr int RB = PackShape<BM, KS, RW>::RB;
  constexpr int XP = PackShape<BM, KS, RW>::XP;
  constexpr int XC = PackShape<BM, KS, RW>::XC;
  constexpr int XBUF = KS * BM * kXRow;             // bytes of one step of x
  constexpr bool XSPARE = XP % kGemmThreads != 0;   // waves past XP load into a spare 1 KB
  static_assert((KS - 1) * RB * RW * CB * 1024 <= kXBufs * XBUF, "the k-slice sums fit the x buffers");
  static_assert(kXBufs * XBUF + (XSPARE ? 1024 : 0) <= 160 * 1024, "x ring fits LDS");
  // Step s reads buffer s % kXBufs, and x(s + kXLead) is loaded into buffer
  // (s - 2) % kXBufs, which step s - 2 read before the last barrier; one
  // array, indexed at run time, so the compiler inserts no waits of its own
  // for these loads (dma_barrier does).
  __shared__ __attribute__((aligned(16))) uint8_t xs[kXBufs * XBUF + (XSPARE ? 1024 : 0)];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / 64);
  const int lane = tid % 64;
  const int col = lane % 16;
  const int grp = lane / 16;
  const int ks = wave % KS;
  const int rb = wave / KS;
  const int nblocks = (a.N + 15) / 16;
  const int kchunks = (a.K + 63) / 64;
  constexpr int HRB = RB / 2;
  static_assert(!SILU || RB % 2 == 0, "gate and up row blocks pair up");
  static_assert(!SILU || (RB / 2) * RW * CB * 64 * 8 <= kXBufs * XBUF, "the up rows' outputs fit the x buffers");
  const int hb = a.N / 32;  // gate row blocks (SILU)
  int nb0;
  if constexpr (SILU) nb0 = rb < HRB ? (blockIdx.x * HRB + rb) * RW : hb + (blockIdx.x * HRB + rb - HRB) * RW;
  else nb0 = (blockIdx.x * RB + rb) * RW;
  const int c0 = blockIdx.y * (a.ksplit / 64);
  const int ce = min(kchunks, c0 + a.ksplit / 64);
  const int m0 = blockIdx.z * BM;
  const int steps = (ce - c0 + KS - 1) / KS;

  const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t*>(a.w), 0, __builtin_amdgcn_readfirstlane(a.w_bytes), kBufferFlags);
  const __amdgpu_buffer_rsrc_t xrsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(a.x), 0, __builtin_amdgcn_readfirstlane(a.x_bytes), kBufferFlags);
  uint32_t woff[RW];
#pragma unroll
  for (int j = 0; j < RW; ++j)
    woff[j] = static_cast<uint32_t>((min(nb0 + j, nblocks - 1) * kchunks + c0 + ks) * 1024 + 16 * lane);
  auto load_w = [&](int s, int j) {
    const bool on = c0 + KS * s + ks < ce;
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                         wrsrc, on ? woff[j] + KS * 1024 * s : kOutOfRange, 0, 0));
  };
  // Piece q = tid + 256 i of a step is token row q / 8 (k slice j, token
  // tok) at LDS position q % 8 of that row, so a wave's 64 pieces fill 1 KB
  // of LDS in lane order, as the LDS-bit load writes them; the swizzle is
  // applied to the source instead (position q % 8 holds chunk x_chunk_at).
  uint32_t xoff[XC];
  int xk[XC];
  bool x_on[XC];
#pragma unroll
  for (int i = 0; i < XC; ++i) {
    const int q = tid + kGemmThreads * i;
    const int j = q / (8 * BM);
    const int tok = (q % (8 * BM)) / 8;
    x_on[i] = q < XP && m0 + tok < a.M;
    xk[i] = 64 * (c0 + j) + 8 * x_chunk_at(tok, q % 8);
    xoff[i] = x_on[i] ? static_cast<uint32_t>(2 * ((m0 + tok) * a.sx + xk[i])) : 0u;
  }
  const int x_end = min(a.K, 64 * ce);
  // Every wave issues XC loads per step, so the counts dma_barrier waits on
  // are the same for all; a wave with no piece in range (XSPARE) writes the
  // zeros its out-of-range loads return into the spare kilobyte.
  auto load_x_lds = [&](int s) {
    uint8_t* buf = xs + (s % kXBufs) * XBUF;
#pragma unroll
    for (int i = 0; i < XC; ++i) {
      const int qw = 64 * wave + kGemmThreads * i;  // the wave's first piece
      uint8_t* dst = (!XSPARE || qw < XP) ? buf + 16 * qw : xs + kXBufs * XBUF;
      const bool on = x_on[i] && xk[i] + 64 * KS * s < x_end;
      buffer_load_lds16(xrsrc, dst, on ? xoff[i] + 2 * 64 * KS * s : kOutOfRange);
    }
  };

  u32x4 wr[kPackRing][RW];
#pragma unroll
  for (int r = 0; r < kPackRing; ++r) {
#pragma unroll
    for (int j = 0; j < RW; ++j) wr[r][j] = load_w(r, j);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int t = 0; t < kXLead; ++t) load_x_lds(t);
  __builtin_amdgcn_sched_barrier(0);

  f32x4 acc[RW][CB];
#pragma unroll
  for (int j = 0; j < RW; ++j)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[j][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int xb_off = (ks * BM + col) * kXRow;  // token rows ks BM + 16 cb + col: low three bits those of col
  const int xc0 = 16 * x_chunk(col, 2 * grp), xc1 = 16 * x_chunk(col, 2 * grp + 1);

  // Weights of the step about to run, already in operand form.
  u32x4 a0[RW], a1[RW];
#pragma unroll
  for (int j = 0; j < RW; ++j) {
    a0[j] = i8x8_to_operand<DT>(wr[0][j][0], wr[0][j][1]);
    a1[j] = i8x8_to_operand<DT>(wr[0][j][2], wr[0][j][3]);
  }
  // x(0) and x(1) in LDS: the loads of x(2) .. x(kXLead - 1) may still be out.
  dma_barrier<(kXLead - 2) * XC>();

  // One step s (ring slot r): read all of x(s) from LDS, refill slot r with
  // weights of step s + kPackRing, then load x(s + kXLead) into LDS, run the
  // MFMAs on the weights converted last step, convert step s + 1's weights
  // while they run, and meet the other waves after odd steps. At that barrier
  // x(s + 1) and x(s + 2) must have landed: the loads issued after them are
  // x(s + 3) .. x(s + kXLead) (XC each) and the weights of the steps since,
  // counted here only for the steps of the current ring pass (NWAIT: a
  // smaller count only waits longer).
  auto step = [&](int s, bool refill, u32x4* wslot, const u32x4* wnext, auto nwait) {
    const uint8_t* xb = xs + (s % kXBufs) * XBUF + xb_off;
    u32x4 b0[CB], b1[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      b0[cb] = *reinterpret_cast<const u32x4*>(xb + cb * 16 * kXRow + xc0);
      b1[cb] = *reinterpret_cast<const u32x4*>(xb + cb * 16 * kXRow + xc1);
    }
    if (refill) {
#pragma unroll
      for (int j = 0; j < RW; ++j) wslot[j] = load_w(s + kPackRing, j);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_x_lds(s + kXLead);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
      for (int j = 0; j < RW; ++j) {
        acc[j][cb] = mfma_16x16x32<DT>(a0[j], b0[cb], acc[j][cb]);
        acc[j][cb] = mfma_16x16x32<DT>(a1[j], b1[cb], acc[j][cb]);
      }
    }
#pragma unroll
    for (int j = 0; j < RW; ++j) {
      a0[j] = i8x8_to_operand<DT>(wnext[j][0], wnext[j][1]);
      a1[j] = i8x8_to_operand<DT>(wnext[j][2], wnext[j][3]);
    }
    if (s & 1) dma_barrier<decltype(nwait)::value>();
  };
  // A ring pass starts on an even step, so its odd steps (r = 1, 3, ...)
  // follow at least two refilling steps of the same pass; the last pass
  // refills nothing.
  static_assert(kPackRing % 2 == 0, "ring passes start on even steps");
  static_assert(kXLead >= 4, "two refilling steps lie between x(s + 2) and an odd step's barrier");
  using WaitRing = std::integral_constant<int, (kXLead - 2) * XC + 2 * RW>;
  using WaitTail = std::integral_constant<int, (kXLead - 2) * XC>;

  int s0 = 0;
  for (; s0 + kPackRing <= steps; s0 += kPackRing) {
#pragma unroll
    for (int r = 0; r < kPackRing; ++r) step(s0 + r, true, wr[r], wr[(r + 1) % kPackRing], WaitRing{});
  }
#pragma unroll
  for (int r = 0; r < kPackRing; ++r) {
    if (s0 + r < steps) step(s0 + r, false, wr[r], wr[(r + 1) % kPackRing], WaitTail{});
  }
  // Every LDS load (those past the last step write zeros) lands before the
  // wave goes on; before LDS is reused below, every wave's.
  wait_vm<0>();
  if constexpr (KS > 1) lds_barrier();

  if constexpr (KS > 1) {
    f32x4* red = reinterpret_cast<f32x4*>(xs);  // [KS - 1][RB][RW][CB][64 lanes]
    if (ks > 0) {
#pragma unroll
      for (int j = 0; j < RW; ++j)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) red[((((ks - 1) * RB + rb) * RW + j) * CB + cb) * 64 + lane] = acc[j][cb];
    }
    lds_barrier();
    if constexpr (!SILU) {
      if (ks > 0) return;
    }
    if (ks == 0) {
#pragma unroll
      for (int t = 1; t < KS; ++t) {
#pragma unroll
        for (int j = 0; j < RW; ++j)
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) acc[j][cb] += red[((((t - 1) * RB + rb) * RW + j) * CB + cb) * 64 + lane];
      }
    }
  }

  if constexpr (SILU) {
    // Every wave reaches both barriers (none has returned); the first also
    // ends the x reads (one k slice) or the k-slice sums' reads of LDS.
    lds_barrier();
    u32x2* ex = reinterpret_cast<u32x2*>(xs);  // [RB/2][RW][CB][64 lanes]: the up rows' outputs
    if (ks == 0 && rb >= HRB) {
#pragma unroll
      for (int j = 0; j < RW; ++j) {
        const int n = 16 * (nb0 + j) + 4 * grp;
        u32x2 sw = u32x2{0u, 0u};
        if (n < a.N) sw = *reinterpret_cast<const u32x2*>(a.scale + n);
        const float sc[4] = {Elem<DT>::to_f32(static_cast<uint16_t>(sw[0])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[0] >> 16)),
                             Elem<DT>::to_f32(static_cast<uint16_t>(sw[1])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[1] >> 16))};
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const f32x4 o = acc[j][cb];
          ex[(((rb - HRB) * RW + j) * CB + cb) * 64 + lane] =
              u32x2{pack2(scaled<DT>(o[0], sc[0]), scaled<DT>(o[1], sc[1])),
                    pack2(scaled<DT>(o[2], sc[2]), scaled<DT>(o[3], sc[3]))};
        }
      }
    }
    lds_barrier();
    if (ks == 0 && rb < HRB) {
#pragma unroll
      for (int j = 0; j < RW; ++j) {
        if (nb0 + j >= hb) continue;  // past the gate half: the tile's last groups
        const int n = 16 * (nb0 + j) + 4 * grp;
        const u32x2 sw = *reinterpret_cast<const u32x2*>(a.scale + n);
        const float sc[4] = {Elem<DT>::to_f32(static_cast<uint16_t>(sw[0])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[0] >> 16)),
                             Elem<DT>::to_f32(static_cast<uint16_t>(sw[1])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[1] >> 16))};
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const int m = m0 + 16 * cb + col;
          if (m < a.M) {
            const f32x4 o = acc[j][cb];
            const u32x2 up = ex[((rb * RW + j) * CB + cb) * 64 + lane];
            uint16_t v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float g = Elem<DT>::to_f32(scaled<DT>(o[e], sc[e]));
              const float u = Elem<DT>::to_f32(static_cast<uint16_t>(up[e / 2] >> (16 * (e % 2))));
              v[e] = silu_mul_value<DT>(g, u);
            }
            *reinterpret_cast<u32x2*>(a.y + static_cast<int64_t>(m) * a.sy + n) = u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
          }
        }
      }
    }
    return;
  }

#pragma unroll
  for (int j = 0; j < RW; ++j) {
    const int n = 16 * (nb0 + j) + 4 * grp;
    if (n >= a.N) continue;
    if (a.splits == 1) {
      const u32x2 sw = *reinterpret_cast<const u32x2*>(a.scale + n);
      const float sc[4] = {Elem<DT>::to_f32(static_cast<uint16_t>(sw[0])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[0] >> 16)),
                           Elem<DT>::to_f32(static_cast<uint16_t>(sw[1])), Elem<DT>::to_f32(static_cast<uint16_t>(sw[1] >> 16))};
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int m = m0 + 16 * cb + col;
        if (m < a.M) {
          const f32x4 o = acc[j][cb];
          const u32x2 v = u32x2{pack2(scaled<DT>(o[0], sc[0]), scaled<DT>(o[1], sc[1])),
                                pack2(scaled<DT>(o[2], sc[2]), scaled<DT>(o[3], sc[3]))};
          *reinterpret_cast<u32x2*>(a.y + static_cast<int64_t>(m) * a.sy + n) = v;
        }
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int m = m0 + 16 * cb + col;
        if (m < a.M) {
          float* p = a.part + (static_cast<int64_t>(blockIdx.y) * a.M + m) * a.N + n;
          *reinterpret_cast<f32x4*>(p) = acc[j][cb];
        }
      }
    }
  }
}

// Packs int8 [N, K] (row stride ws bytes) into the tile order above: one
// thread per 16-byte lane piece of a block.
__global__ __launch_bounds__(256) void int8_pack_kernel(const int8_t* w, int64_t ws, int32_t n, int32_t k,
                                                         int8_t* out) {
  const int64_t kchunks = (k + 63) / 64;
  const int64_t pieces = ((n + 15) / 16) * kchunks * 64;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= pieces) return;
  const int lane = static_cast<int>(idx % 64);
  const int64_t blk = idx / 64;
  const int64_t kc = blk % kchunks;
  const int64_t nb = blk / kchunks;
  const int64_t row = 16 * nb + lane % 16;
  const int64_t k0 = 64 * kc + 16 * (lane / 16);
  uint8_t v[16];
#pragma unroll
  for (int e = 0; e < 16; ++e) v[e] = (row < n && k0 + e < k) ? static_cast<uint8_t>(w[row * ws + k0 + e]) : 0;
  u32x4 o;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    o[d] = static_cast<uint32_t>(v[4 * d]) | (static_cast<uint32_t>(v[4 * d + 1]) << 8) |
           (static_cast<uint32_t>(v[4 * d + 2]) << 16) | (static_cast<uint32_t>(v[4 * d + 3]) << 24);
  }
  *reinterpret_cast<u32x4*>(out + idx * 16) = o;
}

static int64_t packed_bytes(int32_t n, int32_t k) {
  return static_cast<int64_t>((n + 15) / 16) * ((k + 63) / 64) * 1024;
}

// k slices per workgroup: the fewest that still give every CU a workgroup
// (longer per-workgroup streams), but enough row blocks that x, read once
// per workgroup, stays within 2x the weight bytes (16 RB >= BM); then K
// splits if the row tiles alone still leave CUs idle. A pure function of
// the shape.
struct PackPlan {
  int bm, ks, rw;
  int32_t splits, ksplit;
};

static PackPlan packed_plan(int64_t m, int32_t n, int32_t k) {
  PackPlan p;
  p.bm = gemm_bm(m);
  p.rw = 1;
  const int64_t nblocks = (n + 15) / 16;
  const int64_t mtiles = (m + p.bm - 1) / p.bm;
  const int max_ks = kGemmWaves * 16 / p.bm;  // 16 RB >= BM
  p.ks = max_ks;
  for (int ks = 1; ks <= max_ks; ks *= 2) {
    const int rb = kGemmWaves / ks;
    if ((nblocks + rb - 1) / rb * mtiles >= kFillWorkgroups) {
      p.ks = ks;
      break;
    }
  }
  const int rb = kGemmWaves / p.ks;
  const int64_t tiles = (nblocks + rb - 1) / rb * mtiles;
  const int64_t step_k = 64 * p.ks;
  int64_t s = 1;
  if (tiles < kFillWorkgroups) s = (kFillWorkgroups + tiles - 1) / tiles;
  if (s > kMaxSplits) s = kMaxSplits;
  if (s > k / (4 * step_k)) s = k / (4 * step_k);  // at least four steps a split
  if (s < 1) s = 1;
  const int64_t kp = (k + 63) / 64 * 64;
  int64_t ksp = (kp + s - 1) / s;
  ksp = (ksp + step_k - 1) / step_k * step_k;
  p.ksplit = static_cast<int32_t>(ksp);
  p.splits = static_cast<int32_t>((kp + ksp - 1) / ksp);
  return p;
}

template <int DT, int BM, int KS, int RW, bool SILU>
static int launch_packed(const GemmArgs& a, hipStream_t s) {
  constexpr int RB = PackShape<BM, KS, RW>::RB;
  if constexpr (SILU) {
    if constexpr (RB % 2 != 0) {
      return NIMBUS_ERR_UNSUPPORTED;
    } else {
      const int hrw = RB / 2 * RW;
      const dim3 grid((a.N / 32 + hrw - 1) / hrw, 1, (a.M + BM - 1) / BM);
      hipLaunchKernelGGL((int8_matmul_packed_kernel<DT, BM, KS, RW, true>), grid, dim3(kGemmThreads), 0, s, a);
      return static_cast<int>(hipGetLastError());
    }
  }
  const dim3 grid(((a.N + 15) / 16 + RB * RW - 1) / (RB * RW), a.splits, (a.M + BM - 1) / BM);
  hipLaunchKernelGGL((int8_matmul_packed_kernel<DT, BM, KS, RW, false>), grid, dim3(kGemmThreads), 0, s, a);
  if (a.splits > 1 && a.y) {  // (no y: the caller folds the partials in itself)
    const int64_t quads = static_cast<int64_t>(a.M) * (a.N / 4);
    hipLaunchKernelGGL((int8_matmul_reduce_kernel<DT>), dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256),
                       0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

template <int DT, int BM, int KS, bool SILU>
static int launch_packed_rw(const GemmArgs& a, int rw, hipStream_t s) {
  return rw == 2 ? launch_packed<DT, BM, KS, 2, SILU>(a, s) : launch_packed<DT, BM, KS, 1, SILU>(a, s);
}

template <int DT, int BM, bool SILU>
static int launch_packed_bm(const GemmArgs& a, int ks, int rw, hipStream_t s) {
  switch (ks) {
    case 1: return launch_packed_rw<DT, BM, 1, SILU>(a, rw, s);
    case 2: if constexpr (BM <= 64) return launch_packed_rw<DT, BM, 2, SILU>(a, rw, s); else return NIMBUS_ERR_UNSUPPORTED;
    case 4: if constexpr (BM <= 32) return launch_packed_rw<DT, BM, 4, SILU>(a, rw, s); else return NIMBUS_ERR_UNSUPPORTED;
    default:
      if constexpr (BM <= 16 && !SILU) return launch_packed_rw<DT, BM, 8, SILU>(a, rw, s);
      else return NIMBUS_ERR_UNSUPPORTED;
  }
}

template <int DT, bool SILU = false>
static int launch_packed_dt(const GemmArgs& a, const PackPlan& p, hipStream_t s) {
  switch (p.bm) {
    case 16: return launch_packed_bm<DT, 16, SILU>(a, p.ks, p.rw, s);
    case 32: return launch_packed_bm<DT, 32, SILU>(a, p.ks, p.rw, s);
    case 128: return launch_packed_bm<DT, 128, SILU>(a, p.ks, p.rw, s);
    default: return launch_packed_bm<DT, 64, SILU>(a, p.ks, p.rw, s);
  }
}

// Any shape, stride and element alignment: the path of the calls the tiled
// kernels above do not take (n not a multiple of 4, k not a multiple of 16
// (row-major) or 8 (packed), operands past 2 GiB or off their 16-byte
// alignment), as the Triton kernel's masked tiles take any shape. One thread
// per (token, output channel), k summed in order with fp32 FMAs, so equal
// inputs give equal outputs here too; it reads each weight once per token
// and is meant for shapes no model layer has, not for speed.
struct GeneralArgs {
  const uint16_t* x;
  int64_t sx;
  const int8_t* w;
  int64_t sw;  // row stride in bytes (row-major); unused for the packed layout
  const uint16_t* scale;
  uint16_t* y;
  int64_t sy;
  int64_t M;
  int32_t N, K;
};

constexpr int kGeneralThreads = 256;
constexpr int kGeneralRowsMax = 4096;  // grid.y; token rows beyond it are strided

template <bool PACKED>
__device__ __forceinline__ int8_t general_weight(const GeneralArgs& a, int n, int k) {
  if constexpr (PACKED) {
    const int64_t kc = (a.K + 63) / 64;
    const int64_t block = static_cast<int64_t>(n / 16) * kc + k / 64;
    return a.w[block * 1024 + 16 * (16 * ((k % 64) / 16) + n % 16) + k % 16];
  } else {
    return a.w[static_cast<int64_t>(n) * a.sw + k];
  }
}

template <int DT, bool PACKED>
__global__ __launch_bounds__(kGeneralThreads) void int8_matmul_general_kernel(GeneralArgs a) {
  const int n = blockIdx.x * kGeneralThreads + threadIdx.x;
  if (n >= a.N) return;
  const float sc = Elem<DT>::to_f32(a.scale[n]);
  for (int64_t m = blockIdx.y; m < a.M; m += gridDim.y) {
    const uint16_t* xr = a.x + m * a.sx;
    float acc = 0.f;
    for (int k = 0; k < a.K; ++k)
      acc = __builtin_fmaf(Elem<DT>::to_f32(xr[k]), static_cast<float>(general_weight<PACKED>(a, n, k)), acc);
    a.y[m * a.sy + n] = scaled<DT>(acc, sc);
  }
}

template <bool PACKED>
static int launch_general(const GeneralArgs& a, int32_t dtype, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.N + kGeneralThreads - 1) / kGeneralThreads),
                  static_cast<unsigned>(a.M < kGeneralRowsMax ? a.M : kGeneralRowsMax));
  if (dtype == kFloat16) {
    hipLaunchKernelGGL((int8_matmul_general_kernel<kFloat16, PACKED>), grid, dim3(kGeneralThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL((int8_matmul_general_kernel<kBFloat16, PACKED>), grid, dim3(kGeneralThreads), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

static GeneralArgs general_args(const void* x, int64_t x_stride, const void* w, int64_t w_stride, const void* scale,
                                void* y, int64_t y_stride, int64_t m, int32_t n, int32_t k) {
  GeneralArgs g;
  g.x = static_cast<const uint16_t*>(x);
  g.sx = x_stride;
  g.w = static_cast<const int8_t*>(w);
  g.sw = w_stride;
  g.scale = static_cast<const uint16_t*>(scale);
  g.y = static_cast<uint16_t*>(y);
  g.sy = y_stride;
  g.M = m;
  g.N = n;
  g.K = k;
  return g;
}

// Element alignment, the one layout requirement the general kernel has.
static bool elements_aligned(const void* x, const void* scale, const void* y) {
  return ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(scale) | reinterpret_cast<uintptr_t>(y)) %
          2) == 0;
}

// Shapes the tiled kernels take (the workspace queries follow them).
static bool rowmajor_shape_ok(int32_t n, int32_t k) { return n % 4 == 0 && k % 16 == 0; }
static bool packed_shape_ok(int32_t n, int32_t k) { return n % 4 == 0 && k % 8 == 0; }

}  // namespace nimbus

using namespace nimbus;

extern "C" int64_t nimbus_int8_matmul_workspace_bytes(int64_t m, int32_t n, int32_t k) {
  if (m < 0 || n <= 0 || k <= 0) return -1;
  if (!rowmajor_shape_ok(n, k)) return 0;  // the general kernel
  int32_t splits = 1, ksplit = 0;
  gemm_split(m, n, k, &splits, &ksplit);
  return splits > 1 ? static_cast<int64_t>(splits) * m * n * 4 : 0;
}

extern "C" int nimbus_int8_matmul(const void* x, int64_t x_stride, const void* w_q, int64_t w_stride,
                                  const void* scale, void* y, int64_t y_stride, int64_t m, int32_t n, int32_t k,
                                  void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (m == 0) return NIMBUS_OK;
  if (!x || !w_q || !scale || !y) return NIMBUS_ERR_INVALID;
  if (x_stride < k || w_stride < k || y_stride < n) return NIMBUS_ERR_INVALID;
  if (!elements_aligned(x, scale, y)) return NIMBUS_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The tiled kernel: token tiles fit grid.z, buffer offsets are 32-bit (each
  // operand under 2 GiB), 16-byte rows and operands.
  const int64_t x_bytes = ((m - 1) * x_stride + k) * 2;
  const int64_t w_bytes = (static_cast<int64_t>(n) - 1) * w_stride + k;
  const bool tiled = rowmajor_shape_ok(n, k) && m <= (int64_t{1} << 21) && x_bytes < (int64_t{1} << 31) &&
                     w_bytes < (int64_t{1} << 31) && x_stride % 8 == 0 && w_stride % 16 == 0 && y_stride % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_q) |
                      reinterpret_cast<uintptr_t>(y)) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(scale) % 8 == 0;
  if (!tiled)
    return launch_general<false>(general_args(x, x_stride, w_q, w_stride, scale, y, y_stride, m, n, k), dtype, s);
  GemmArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.sx = static_cast<int32_t>(x_stride);
  a.w = static_cast<const int8_t*>(w_q);
  a.sw = static_cast<int32_t>(w_stride);
  a.x_bytes = static_cast<int32_t>(x_bytes);
  a.w_bytes = static_cast<int32_t>(w_bytes);
  a.scale = static_cast<const uint16_t*>(scale);
  a.y = static_cast<uint16_t*>(y);
  a.sy = y_stride;
  a.M = static_cast<int32_t>(m);
  a.N = n;
  a.K = k;
  gemm_split(m, n, k, &a.splits, &a.ksplit);
  const int64_t need = a.splits > 1 ? static_cast<int64_t>(a.splits) * m * n * 4 : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return NIMBUS_ERR_WORKSPACE;
  if (need > 0 && reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return NIMBUS_ERR_ALIGNMENT;
  a.part = static_cast<float*>(workspace);
  return dtype == kFloat16 ? launch_gemm_dt<kFloat16>(a, s) : launch_gemm_dt<kBFloat16>(a, s);
}

extern "C" int64_t nimbus_int8_packed_weight_bytes(int32_t n, int32_t k) {
  if (n <= 0 || k <= 0) return -1;
  return packed_bytes(n, k);
}

extern "C" int nimbus_int8_pack_weight(const void* w_q, int64_t w_stride, int32_t n, int32_t k, void* out,
                                       void* stream) {
  if (n <= 0 || k <= 0 || w_stride < k) return NIMBUS_ERR_INVALID;
  if (!w_q || !out) return NIMBUS_ERR_INVALID;
  if (reinterpret_cast<uintptr_t>(out) % 16 != 0) return NIMBUS_ERR_ALIGNMENT;
  const int64_t pieces = packed_bytes(n, k) / 16;
  hipLaunchKernelGGL(int8_pack_kernel, dim3(static_cast<unsigned>((pieces + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const int8_t*>(w_q), w_stride, n, k,
                     static_cast<int8_t*>(out));
  return static_cast<int>(hipGetLastError());
}

extern "C" int64_t nimbus_int8_matmul_packed_workspace_bytes(int64_t m, int32_t n, int32_t k) {
  if (m < 0 || n <= 0 || k <= 0) return -1;
  if (!packed_shape_ok(n, k)) return 0;  // the general kernel
  const PackPlan p = packed_plan(m, n, k);
  return p.splits > 1 ? static_cast<int64_t>(p.splits) * m * n * 4 : 0;
}

static int packed_impl(const void* x, int64_t x_stride, const void* w_packed, const void* scale, void* y,
                       int64_t y_stride, int64_t m, int32_t n, int32_t k, const PackPlan* forced, void* workspace,
                       int64_t workspace_bytes, int32_t dtype, void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (forced && !packed_shape_ok(n, k)) return NIMBUS_ERR_UNSUPPORTED;  // plans are the tiled kernel's
  if (m == 0) return NIMBUS_OK;
  if (!x || !w_packed || !scale || !y) return NIMBUS_ERR_INVALID;
  if (x_stride < k || y_stride < n) return NIMBUS_ERR_INVALID;
  if (!elements_aligned(x, scale, y)) return NIMBUS_ERR_ALIGNMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t x_bytes = ((m - 1) * x_stride + k) * 2;
  const int64_t w_bytes = packed_bytes(n, k);
  const bool tiled = packed_shape_ok(n, k) && m <= (int64_t{1} << 21) && x_bytes < (int64_t{1} << 31) &&
                     w_bytes < (int64_t{1} << 31) && x_stride % 8 == 0 && y_stride % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_packed) |
                      reinterpret_cast<uintptr_t>(y)) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(scale) % 8 == 0;
  if (!tiled) {
    if (forced) {
      const bool too_big = m > (int64_t{1} << 21) || x_bytes >= (int64_t{1} << 31) || w_bytes >= (int64_t{1} << 31);
      return too_big ? NIMBUS_ERR_UNSUPPORTED : NIMBUS_ERR_ALIGNMENT;
    }
    return launch_general<true>(general_args(x, x_stride, w_packed, 0, scale, y, y_stride, m, n, k), dtype, s);
  }
  GemmArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.sx = static_cast<int32_t>(x_stride);
  a.w = static_cast<const int8_t*>(w_packed);
  a.sw = 0;
  a.x_bytes = static_cast<int32_t>(x_bytes);
  a.w_bytes = static_cast<int32_t>(w_bytes);
  a.scale = static_cast<const uint16_t*>(scale);
  a.y = static_cast<uint16_t*>(y);
  a.sy = y_stride;
  a.M = static_cast<int32_t>(m);
  a.N = n;
  a.K = k;
  const PackPlan plan = forced ? *forced : packed_plan(m, n, k);
  a.splits = plan.splits;
  a.ksplit = plan.ksplit;
  const int64_t need = a.splits > 1 ? static_cast<int64_t>(a.splits) * m * n * 4 : 0;
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) return NIMBUS_ERR_WORKSPACE;
  if (need > 0 && reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return NIMBUS_ERR_ALIGNMENT;
  a.part = static_cast<float*>(workspace);
  return dtype == kFloat16 ? launch_packed_dt<kFloat16>(a, plan, s) : launch_packed_dt<kBFloat16>(a, plan, s);
}

extern "C" int nimbus_int8_matmul_packed(const void* x, int64_t x_stride, const void* w_packed, const void* scale,
                                         void* y, int64_t y_stride, int64_t m, int32_t n, int32_t k,
                                         void* workspace, int64_t workspace_bytes, int32_t dtype, void* stream) {
  return packed_impl(x, x_stride, w_packed, scale, y, y_stride, m, n, k, nullptr, workspace, workspace_bytes, dtype,
                     stream);
}

// An explicit plan: token tile bm (16, 32, 64, 128), k slices ks (1, 2, 4,
// 8; ks * bm <= 128), k splits (1..16, fewer when K is short) and row blocks
// per wave rw (1, 2). Its token tiles are the grid's z dimension, so there
// are at most 65535 of them. Workspace: splits * m * n * 4 bytes when the
// plan splits.
static bool make_plan(int64_t m, int32_t n, int32_t k, int32_t bm, int32_t ks, int32_t splits, int32_t rw,
                      PackPlan* p) {
  (void)n;
  if (bm != 16 && bm != 32 && bm != 64 && bm != 128) return false;
  if ((m + bm - 1) / bm > 65535) return false;
  if (ks != 1 && ks != 2 && ks != 4 && ks != 8) return false;
  if (rw != 1 && rw != 2) return false;
  if (ks * bm > 128 || splits < 1 || splits > kMaxSplits) return false;
  const int64_t step_k = 64 * ks;
  const int64_t kp = (k + 63) / 64 * 64;
  int64_t ksp = (kp + splits - 1) / splits;
  ksp = (ksp + step_k - 1) / step_k * step_k;
  p->bm = bm;
  p->ks = ks;
  p->rw = rw;
  p->ksplit = static_cast<int32_t>(ksp);
  p->splits = static_cast<int32_t>((kp + ksp - 1) / ksp);
  return true;
}

extern "C" int64_t nimbus_int8_matmul_packed_plan_workspace_bytes(int64_t m, int32_t n, int32_t k, int32_t bm,
                                                                  int32_t ks, int32_t splits,
                                                                  int32_t rows_per_wave) {
  PackPlan p;
  if (m < 0 || n <= 0 || k <= 0 || !packed_shape_ok(n, k) || !make_plan(m, n, k, bm, ks, splits, rows_per_wave, &p))
    return -1;
  return p.splits > 1 ? static_cast<int64_t>(p.splits) * m * n * 4 : 0;
}

extern "C" int nimbus_int8_matmul_packed_plan(const void* x, int64_t x_stride, const void* w_packed,
                                              const void* scale, void* y, int64_t y_stride, int64_t m, int32_t n,
                                              int32_t k, int32_t bm, int32_t ks, int32_t splits,
                                              int32_t rows_per_wave, void* workspace, int64_t workspace_bytes,
                                              int32_t dtype, void* stream) {
  PackPlan p;
  if (m < 0 || n <= 0 || k <= 0) return NIMBUS_ERR_INVALID;
  if (!make_plan(m, n, k, bm, ks, splits, rows_per_wave, &p)) return NIMBUS_ERR_UNSUPPORTED;
  return packed_impl(x, x_stride, w_packed, scale, y, y_stride, m, n, k, &p, workspace, workspace_bytes, dtype,
                     stream);
}

// Llama's gate_up projection fused with its SiLU gate: y [m, n/2] =
// silu(gate) * up of the projection's outputs gate = [:, :n/2], up =
// [:, n/2:] (each rounded to the model dtype first, as the projection would
// store them), without writing the projection's output. A plan of one split
// (bm, ks in 1, 2, 4, rows_per_wave); bm = 0 takes bm from m, one k slice,
// one row block per wave.
extern "C" int nimbus_int8_matmul_packed_silu(const void* x, int64_t x_stride, const void* w_packed,
                                              const void* scale, void* y, int64_t y_stride, int64_t m, int32_t n,
                                              int32_t k, int32_t bm, int32_t ks, int32_t rows_per_wave,
                                              int32_t dtype, void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (n % 32 != 0 || !packed_shape_ok(n, k)) return NIMBUS_ERR_UNSUPPORTED;
  if (bm == 0) {
    bm = gemm_bm(m);
    ks = 1;
    rows_per_wave = 1;
  }
  PackPlan p;
  if (ks == 8 || !make_plan(m, n, k, bm, ks, 1, rows_per_wave, &p) || p.splits != 1) return NIMBUS_ERR_UNSUPPORTED;
  if (m == 0) return NIMBUS_OK;
  if (!x || !w_packed || !scale || !y) return NIMBUS_ERR_INVALID;
  if (x_stride < k || y_stride < n / 2) return NIMBUS_ERR_INVALID;
  if (!elements_aligned(x, scale, y)) return NIMBUS_ERR_ALIGNMENT;
  const int64_t x_bytes = ((m - 1) * x_stride + k) * 2;
  const int64_t w_bytes = packed_bytes(n, k);
  if (m > (int64_t{1} << 21) || x_bytes >= (int64_t{1} << 31) || w_bytes >= (int64_t{1} << 31))
    return NIMBUS_ERR_UNSUPPORTED;
  if (x_stride % 8 != 0 || y_stride % 4 != 0 ||
      (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_packed) | reinterpret_cast<uintptr_t>(y)) %
              16 != 0 ||
      reinterpret_cast<uintptr_t>(scale) % 8 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  GemmArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.sx = static_cast<int32_t>(x_stride);
  a.w = static_cast<const int8_t*>(w_packed);
  a.sw = 0;
  a.x_bytes = static_cast<int32_t>(x_bytes);
  a.w_bytes = static_cast<int32_t>(w_bytes);
  a.scale = static_cast<const uint16_t*>(scale);
  a.y = static_cast<uint16_t*>(y);
  a.sy = y_stride;
  a.part = nullptr;
  a.M = static_cast<int32_t>(m);
  a.N = n;
  a.K = k;
  a.splits = 1;
  a.ksplit = p.ksplit;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == kFloat16 ? launch_packed_dt<kFloat16, true>(a, p, s) : launch_packed_dt<kBFloat16, true>(a, p, s);
}

// The split-K partials of a packed-weight projection, without the reducing
// launch: workspace [splits][m][n] fp32 receives each split's sum over its
// part of K, in the layout int8_matmul_reduce_kernel reads, for a consumer
// that folds them in itself (nimbus_add_rms_norm_partials). The plan must
// split K (splits >= 2 after make_plan).
extern "C" int nimbus_int8_matmul_packed_partials(const void* x, int64_t x_stride, const void* w_packed, int64_t m,
                                                  int32_t n, int32_t k, int32_t bm, int32_t ks, int32_t splits,
                                                  int32_t rows_per_wave, void* workspace, int64_t workspace_bytes,
                                                  int32_t dtype, void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  PackPlan p;
  if (!packed_shape_ok(n, k) || !make_plan(m, n, k, bm, ks, splits, rows_per_wave, &p) || p.splits < 2)
    return NIMBUS_ERR_UNSUPPORTED;
  if (m == 0) return NIMBUS_OK;
  if (!x || !w_packed) return NIMBUS_ERR_INVALID;
  if (x_stride < k) return NIMBUS_ERR_INVALID;
  const int64_t x_bytes = ((m - 1) * x_stride + k) * 2;
  const int64_t w_bytes = packed_bytes(n, k);
  if (m > (int64_t{1} << 21) || x_bytes >= (int64_t{1} << 31) || w_bytes >= (int64_t{1} << 31))
    return NIMBUS_ERR_UNSUPPORTED;
  if (x_stride % 8 != 0 || (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w_packed)) % 16 != 0)
    return NIMBUS_ERR_ALIGNMENT;
  const int64_t need = static_cast<int64_t>(p.splits) * m * n * 4;
  if (workspace == nullptr || workspace_bytes < need) return NIMBUS_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return NIMBUS_ERR_ALIGNMENT;
  GemmArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.sx = static_cast<int32_t>(x_stride);
  a.w = static_cast<const int8_t*>(w_packed);
  a.sw = 0;
  a.x_bytes = static_cast<int32_t>(x_bytes);
  a.w_bytes = static_cast<int32_t>(w_bytes);
  a.scale = nullptr;
  a.y = nullptr;
  a.sy = 0;
  a.part = static_cast<float*>(workspace);
  a.M = static_cast<int32_t>(m);
  a.N = n;
  a.K = k;
  a.splits = p.splits;
  a.ksplit = p.ksplit;
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == kFloat16 ? launch_packed_dt<kFloat16, false>(a, p, s) : launch_packed_dt<kBFloat16, false>(a, p, s);
}
