// Fused residual add + RMSNorm for gfx950.
//
// Replaces nimbus/kernels/rmsnorm.py:21-59 (the Triton _rmsnorm_kernel and
// its rms_norm / add_rms_norm wrappers). Numerics follow
// nimbus/kernels/reference.py:99-112 (HuggingFace's LlamaRMSNorm):
//   s   = x + r                      in the model dtype (the new residual)
//   y   = dtype(s * rsqrt(mean(s^2) + eps))   mean and scale in fp32
//   out = dtype(w * y)               the weight multiply in the model dtype
//
// 256-thread workgroups (four waves; a measured 1.1-1.4x over one wave per row
// at 2k-4k columns, and two waves per row measured 18% slower at 2108 x 4096)
// that walk rows with the next row's loads in flight. A lane owns 16-byte chunks of its row:
// every load and store of a wave is 1 KB contiguous. The row is read once (x,
// and r when fused), the rounded sum stays in registers for the second pass,
// and the sum of squares is reduced across each wave with lane shuffles and
// across the four waves through LDS.
// HBM traffic per row: read x (and r), write out (and the new residual); the
// weight is read by every row but stays in L2.
#include "common.h"
#include "int8_epilogue.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

constexpr int kNormMaxChunksPerLane = 4;  // cols <= 256 * 4 * 8 = 8192

struct NormArgs {
  const uint16_t* x;
  int64_t sx;
  const uint16_t* r;  // null: plain RMSNorm
  int64_t sr;
  const uint16_t* w;
  uint16_t* out;
  int64_t so;
  uint16_t* rout;
  int64_t sro;
  int32_t rows, cols;
  float eps;
  // PART: x is an INT8 projection's split-K partials, [splits][rows][cols]
  // fp32, folded in here as its reducing launch would: summed in split order,
  // times the channel scale, rounded to the model dtype.
  const float* part;
  int64_t plane;
  int32_t splits;
  const uint16_t* pscale;
};

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h16x2 __attribute__((ext_vector_type(2)));

// Two packed elements <-> two fp32 values (round to nearest even).
template <int DT>
__device__ __forceinline__ f32x2 unpack_pair(uint32_t w);
template <>
__device__ __forceinline__ f32x2 unpack_pair<kFloat16>(uint32_t w) {
  return __builtin_convertvector(__builtin_bit_cast(h16x2, w), f32x2);
}
template <>
__device__ __forceinline__ f32x2 unpack_pair<kBFloat16>(uint32_t w) {
  return f32x2{__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
}
template <int DT>
__device__ __forceinline__ uint32_t pack_pair(f32x2 v);
template <>
__device__ __forceinline__ uint32_t pack_pair<kFloat16>(f32x2 v) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h16x2));
}
template <>
__device__ __forceinline__ uint32_t pack_pair<kBFloat16>(f32x2 v) {
  return pack2(f32_to_bf16(v[0]), f32_to_bf16(v[1]));
}

// Workgroups of four waves walk rows blockIdx.x, + gridDim.x, ... (one row
// each when the grid covers the rows). Lane l of wave wr owns the row's
// 16-byte chunks c = l + 64 (wr + 4 i), i < NCH; the weight is loaded once.
// The next row's x and r are loaded before the current row's output is
// stored, so a workgroup's reads and writes overlap. The new residual's
// stores may alias the inputs as far as the compiler knows, so they stay
// after the loads of the row they belong to (interleaving them would
// serialise the round trips). Stores are nontemporal (streamed past the L2;
// nothing here reads them again): 8.2 -> 6.9 us at 2048 x 2048 fp16,
// unchanged at 2108 x 4096 bf16 and 64 rows.
constexpr int kFold = 4;  // split-K partials of a chunk loaded at once (PART)

template <int DT, int NCH, bool RES, bool PART>
__global__ __launch_bounds__(256) void add_rms_norm_kernel(NormArgs a) {
  const int wave = static_cast<int>(threadIdx.x) / 64;
  const int lane = threadIdx.x % 64;
  const int nchunk = a.cols / 8;
  u32x4 ww[NCH], xw[NCH], rw[NCH];
  bool on[NCH];
  int cidx[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    cidx[c] = lane + 64 * (wave + 4 * c);
    on[c] = cidx[c] < nchunk;
    if (on[c]) ww[c] = *reinterpret_cast<const u32x4*>(a.w + 8 * cidx[c]);
  }
  auto load = [&](int row) {
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (on[c]) {
        if constexpr (!PART) xw[c] = *reinterpret_cast<const u32x4*>(a.x + static_cast<int64_t>(row) * a.sx + 8 * cidx[c]);
        if constexpr (RES) rw[c] = *reinterpret_cast<const u32x4*>(a.r + static_cast<int64_t>(row) * a.sr + 8 * cidx[c]);
      }
    }
    if constexpr (PART) {
      // The projection's output chunks, bit for bit as its reducing launch
      // would store them (int8_matmul_reduce_kernel: the splits summed in
      // order, times the scale, rounded). kFold splits' loads of every chunk
      // go out together before any is added: one load round trip per kFold
      // splits instead of per split (64 x 4096 bf16, per call in a graph of
      // back-to-back calls: 4 splits 6.85 -> 6.17 us, 8 splits 11.4 -> 9.3 us;
      // the plain norm 4.2 us, the reducing launch this replaces ~4.5 us).
      const float* base = a.part + static_cast<int64_t>(row) * a.cols;
      f32x4 lo[NCH], hi[NCH];
      for (int k0 = 0; k0 < a.splits; k0 += kFold) {
        f32x4 l[NCH][kFold], h[NCH][kFold];
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
          for (int j = 0; j < kFold; ++j) {
            if (on[c] && k0 + j < a.splits) {
              const float* p = base + (k0 + j) * a.plane + 8 * cidx[c];
              l[c][j] = *reinterpret_cast<const f32x4*>(p);
              h[c][j] = *reinterpret_cast<const f32x4*>(p + 4);
            }
          }
        }
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
#pragma unroll
          for (int j = 0; j < kFold; ++j) {
            if (on[c] && k0 + j < a.splits) {
              if (k0 + j == 0) {
                lo[c] = l[c][j];
                hi[c] = h[c][j];
              } else {
                lo[c] += l[c][j];
                hi[c] += h[c][j];
              }
            }
          }
        }
      }
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        if (on[c]) {
          const u32x4 sw = *reinterpret_cast<const u32x4*>(a.pscale + 8 * cidx[c]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const f32x4& v = e < 2 ? lo[c] : hi[c];
            const int i = 2 * (e % 2);
            xw[c][e] = pack2(scaled<DT>(v[i], Elem<DT>::to_f32(static_cast<uint16_t>(sw[e]))),
                             scaled<DT>(v[i + 1], Elem<DT>::to_f32(static_cast<uint16_t>(sw[e] >> 16))));
          }
        }
      }
    }
  };
  // Partial sums per wave, double-buffered: a wave that runs ahead writes the
  // other half while the slowest still reads this row's (the next reuse of a
  // half is two rows on, past the next row's barrier).
  __shared__ float part[2][4];
  int par = 0;
  int row = blockIdx.x;
  if (row < a.rows) load(row);
  for (; row < a.rows; row += gridDim.x) {
    f32x2 v[NCH][4];
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (on[c]) {
        if constexpr (RES) {
          u32x4 sw;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // The exact sum of two fp16 (or bf16) values fits fp32, so one
            // rounding to the element type is the model dtype's own add.
            sw[e] = pack_pair<DT>(unpack_pair<DT>(xw[c][e]) + unpack_pair<DT>(rw[c][e]));
            v[c][e] = unpack_pair<DT>(sw[e]);
          }
          __builtin_nontemporal_store(
              sw, reinterpret_cast<u32x4*>(a.rout + static_cast<int64_t>(row) * a.sro + 8 * cidx[c]));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[c][e] = unpack_pair<DT>(xw[c][e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ss = __builtin_fmaf(v[c][e][0], v[c][e][0], ss);
          ss = __builtin_fmaf(v[c][e][1], v[c][e][1], ss);
        }
      }
    }
    const int next = row + static_cast<int>(gridDim.x);
    if (next < a.rows) load(next);
    ss = wave_sum(ss);
    if (lane == 0) part[par][wave] = ss;
    __syncthreads();
    ss = (part[par][0] + part[par][1]) + (part[par][2] + part[par][3]);
    par ^= 1;
    const float inv = 1.f / __builtin_sqrtf(ss / static_cast<float>(a.cols) + a.eps);

    uint16_t* orow = a.out + static_cast<int64_t>(row) * a.so;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (on[c]) {
        u32x4 ow;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const f32x2 y = unpack_pair<DT>(pack_pair<DT>(v[c][e] * inv));  // dtype(s * rsqrt(...))
          ow[e] = pack_pair<DT>(unpack_pair<DT>(ww[c][e]) * y);
        }
        __builtin_nontemporal_store(ow, reinterpret_cast<u32x4*>(orow + 8 * cidx[c]));
      }
    }
  }
}

// Workgroups in flight: six per CU of a 256-CU part (the register budget
// holds six four-wave workgroups per CU up to 4096 columns, four at 8192).
// Measured against one workgroup per row (hipGraph of back-to-back calls,
// alternated three times on one box): 2048 x 2048 fp16 6.50-6.55 us against
// 6.86-6.92, 64 x 4096 bf16 4.08 against 4.35, 4096 x 4096 bf16 27.5-27.8
// against 27.9-28.3, 2108 x 4096 bf16 16.9-17.4 against 17.2; grids of 512
// to 1024 workgroups measured no better or slower.
constexpr int kNormGrid = 1536;

template <int DT, int NCH>
static int launch_norm_nch(const NormArgs& a, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(a.rows < kNormGrid ? a.rows : kNormGrid);
  if (a.part) {
    hipLaunchKernelGGL((add_rms_norm_kernel<DT, NCH, true, true>), dim3(grid), dim3(256), 0, s, a);
  } else if (a.r) {
    hipLaunchKernelGGL((add_rms_norm_kernel<DT, NCH, true, false>), dim3(grid), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((add_rms_norm_kernel<DT, NCH, false, false>), dim3(grid), dim3(256), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

template <int DT>
static int launch_norm(const NormArgs& a, hipStream_t s) {
  switch ((a.cols / 8 + 255) / 256) {  // chunks per lane
    case 1: return launch_norm_nch<DT, 1>(a, s);
    case 2: return launch_norm_nch<DT, 2>(a, s);
    default: return launch_norm_nch<DT, kNormMaxChunksPerLane>(a, s);
  }
}

// Any row length, stride and element alignment: the path of the calls the
// chunked kernel above does not take (a row length not a multiple of 8 or
// past 8192, rows off their 16-byte alignment), as the Triton kernel's
// masked block takes any row. One 256-thread workgroup per row at a time,
// an element per thread per pass: the sum of squares of the rounded sums,
// reduced as above, then a second pass that writes the output. With a
// residual, the second pass reads back the rounded sum the first pass stored
// in residual_out (the same thread wrote it): residual_out may then alias x
// or the residual, as it may in the chunked kernel, since every element is
// read before it is written and by the thread that writes it.
template <int DT>
__device__ __forceinline__ float elem_f32(uint16_t v) {
  return Elem<DT>::to_f32(v);
}

template <int DT, bool RES>
__global__ __launch_bounds__(256) void add_rms_norm_general_kernel(NormArgs a) {
  const int wave = static_cast<int>(threadIdx.x) / 64;
  const int lane = threadIdx.x % 64;
  __shared__ float part[2][4];
  int par = 0;
  auto sum_at = [&](int64_t row, int c) {  // dtype(x + r), as a float
    const float xv = elem_f32<DT>(a.x[row * a.sx + c]);
    if constexpr (RES) return elem_f32<DT>(Elem<DT>::from_f32(xv + elem_f32<DT>(a.r[row * a.sr + c])));
    else return xv;
  };
  for (int row = blockIdx.x; row < a.rows; row += gridDim.x) {
    float ss = 0.f;
    for (int c = threadIdx.x; c < a.cols; c += 256) {
      const float v = sum_at(row, c);
      if constexpr (RES) a.rout[static_cast<int64_t>(row) * a.sro + c] = Elem<DT>::from_f32(v);
      ss = __builtin_fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if (lane == 0) part[par][wave] = ss;
    __syncthreads();
    ss = (part[par][0] + part[par][1]) + (part[par][2] + part[par][3]);
    par ^= 1;
    const float inv = 1.f / __builtin_sqrtf(ss / static_cast<float>(a.cols) + a.eps);
    for (int c = threadIdx.x; c < a.cols; c += 256) {
      float v;
      if constexpr (RES) v = elem_f32<DT>(a.rout[static_cast<int64_t>(row) * a.sro + c]);
      else v = sum_at(row, c);
      const float y = elem_f32<DT>(Elem<DT>::from_f32(v * inv));  // dtype(s * rsqrt(...))
      a.out[static_cast<int64_t>(row) * a.so + c] = Elem<DT>::from_f32(elem_f32<DT>(a.w[c]) * y);
    }
  }
}

template <int DT>
static int launch_norm_general(const NormArgs& a, hipStream_t s) {
  const unsigned grid = static_cast<unsigned>(a.rows < kNormGrid ? a.rows : kNormGrid);
  if (a.r) {
    hipLaunchKernelGGL((add_rms_norm_general_kernel<DT, true>), dim3(grid), dim3(256), 0, s, a);
  } else {
    hipLaunchKernelGGL((add_rms_norm_general_kernel<DT, false>), dim3(grid), dim3(256), 0, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

}  // namespace nimbus

using namespace nimbus;

extern "C" int nimbus_add_rms_norm(const void* x, int64_t x_stride, const void* residual, int64_t residual_stride,
                                   const void* weight, void* out, int64_t out_stride, void* residual_out,
                                   int64_t residual_out_stride, int64_t rows, int32_t cols, float eps, int32_t dtype,
                                   void* stream) {
  if (rows < 0 || cols <= 0) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (rows > INT32_MAX) return NIMBUS_ERR_UNSUPPORTED;
  if (rows == 0) return NIMBUS_OK;
  if (!x || !weight || !out || (residual && !residual_out)) return NIMBUS_ERR_INVALID;
  const uintptr_t ptrs = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
                         reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual) |
                         reinterpret_cast<uintptr_t>(residual_out);
  if (ptrs % 2 != 0) return NIMBUS_ERR_ALIGNMENT;  // 2-byte elements
  // The chunked kernel: rows of 16-byte chunks, at most 8192 elements.
  const bool chunked = cols % 8 == 0 && cols <= 256 * kNormMaxChunksPerLane * 8 && ptrs % 16 == 0 &&
                       (x_stride | out_stride | (residual ? residual_stride | residual_out_stride : 0)) % 8 == 0;
  NormArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.sx = x_stride;
  a.r = static_cast<const uint16_t*>(residual);
  a.sr = residual_stride;
  a.w = static_cast<const uint16_t*>(weight);
  a.out = static_cast<uint16_t*>(out);
  a.so = out_stride;
  a.rout = static_cast<uint16_t*>(residual_out);
  a.sro = residual_out_stride;
  a.rows = static_cast<int32_t>(rows);
  a.cols = cols;
  a.eps = eps;
  a.part = nullptr;
  a.plane = 0;
  a.splits = 0;
  a.pscale = nullptr;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (!chunked) return dtype == kFloat16 ? launch_norm_general<kFloat16>(a, s) : launch_norm_general<kBFloat16>(a, s);
  return dtype == kFloat16 ? launch_norm<kFloat16>(a, s) : launch_norm<kBFloat16>(a, s);
}

extern "C" int nimbus_add_rms_norm_partials(const float* partials, int32_t splits, const void* scale,
                                            const void* residual, int64_t residual_stride, const void* weight,
                                            void* out, int64_t out_stride, void* residual_out,
                                            int64_t residual_out_stride, int64_t rows, int32_t cols, float eps,
                                            int32_t dtype, void* stream) {
  if (rows < 0 || cols <= 0 || splits < 1) return NIMBUS_ERR_INVALID;
  if (dtype != kFloat16 && dtype != kBFloat16) return NIMBUS_ERR_UNSUPPORTED;
  if (rows > INT32_MAX || cols % 8 != 0 || cols > 256 * kNormMaxChunksPerLane * 8) return NIMBUS_ERR_UNSUPPORTED;
  if (rows == 0) return NIMBUS_OK;
  if (!partials || !scale || !residual || !weight || !out || !residual_out) return NIMBUS_ERR_INVALID;
  if (residual_stride < cols || out_stride < cols || residual_out_stride < cols) return NIMBUS_ERR_INVALID;
  const uintptr_t ptrs = reinterpret_cast<uintptr_t>(partials) | reinterpret_cast<uintptr_t>(scale) |
                         reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(weight) |
                         reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual_out);
  if (ptrs % 16 != 0 || (residual_stride | out_stride | residual_out_stride) % 8 != 0) return NIMBUS_ERR_ALIGNMENT;
  NormArgs a;
  a.x = nullptr;
  a.sx = 0;
  a.r = static_cast<const uint16_t*>(residual);
  a.sr = residual_stride;
  a.w = static_cast<const uint16_t*>(weight);
  a.out = static_cast<uint16_t*>(out);
  a.so = out_stride;
  a.rout = static_cast<uint16_t*>(residual_out);
  a.sro = residual_out_stride;
  a.rows = static_cast<int32_t>(rows);
  a.cols = cols;
  a.eps = eps;
  a.part = partials;
  a.plane = rows * cols;
  a.splits = splits;
  a.pscale = static_cast<const uint16_t*>(scale);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == kFloat16 ? launch_norm<kFloat16>(a, s) : launch_norm<kBFloat16>(a, s);
}
