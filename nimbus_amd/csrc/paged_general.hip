// Paged attention for the shapes the tuned kernels do not take: any page
// (block) size and any head dim up to 256.
//
// The reference's Triton kernels take BLOCK_SIZE = k_cache.shape[1] and any
// power-of-two head dim (nimbus/kernels/paged_attention.py:35-80, 139-140;
// nimbus/kernels/prefill_attention.py:27-78, 115), while
// paged_decode_kernel and paged_prefill_kernel are built for 16-token pages
// and D = 64 or 128. Shapes outside those run here instead of being refused,
// as the reference's masked tiles run them: correct, not tuned (no model
// layer of the benchmarked families takes this path).
//
// One workgroup per (query row, kv head, chunk of that kv head's query
// heads): the query row is a decode sequence (or one query of a verify
// call's sequence, which sees keys up to its own position) or one position
// of a prefill tile. It walks the row's visible keys kGenTile at a time through
// LDS in fp32: K and V rows of the tile gathered through the block table
// (page = table[key / block_size], row key % block_size; page ids outside
// [0, num_blocks) read page 0, as in the tuned kernels), scores for every
// (head, key), an online softmax per head (exp2 domain, running max from a
// finite floor so that a row with no visible key gives 0), and O
// accumulated in LDS. P and V stay fp32 (the products are exact to fp32
// rounding; the reference computes them in fp32 as well).
#include "common.h"
#include "nimbus_attn_internal.h"

namespace nimbus {

constexpr int kGenThreads = 256;
constexpr int kGenTile = 16;  // keys per LDS tile

template <int DT, bool PREFILL>
__global__ __launch_bounds__(kGenThreads) void paged_general_kernel(AttnGeneralArgs a) {
  extern __shared__ float lds[];
  const int D = a.D;
  const int gc = a.gc;
  float* qs = lds;                      // [gc][D] q * scale * log2(e)
  float* acc = qs + gc * D;             // [gc][D]
  float* kt = acc + gc * D;             // [kGenTile][D]
  float* vt = kt + kGenTile * D;        // [kGenTile][D]
  float* sc = vt + kGenTile * D;        // [gc][kGenTile] scores, then weights
  float* mrun = sc + gc * kGenTile;     // [gc]
  float* lrun = mrun + gc;              // [gc]
  float* alpha = lrun + gc;             // [gc]
  const int tid = threadIdx.x;

  // The row: its sequence, output token and number of visible keys.
  int seq, tok, limit;
  if constexpr (PREFILL) {
    const int tile = blockIdx.x / a.tile_pos;
    const int pos = a.prog_m[tile] + blockIdx.x % a.tile_pos;
    seq = a.prog_seq[tile];
    const int q0 = a.qstart[seq];
    const int q_len = a.qstart[seq + 1] - q0;
    if (pos >= q_len) return;
    tok = q0 + pos;
    limit = a.ctx[seq] - q_len + pos + 1;  // keys 0 .. ctx - q_len + pos
  } else {
    seq = blockIdx.x / a.nq;
    const int j = blockIdx.x % a.nq;
    tok = blockIdx.x;
    limit = min(a.ctx[seq], a.max_ctx) - (a.nq - 1 - j);
  }
  limit = min(limit, a.bt_width * a.bs);  // the block table bounds the readable keys
  const int kvh = blockIdx.y / a.nchunks;
  const int g0 = (blockIdx.y % a.nchunks) * gc;
  const int ng = min(gc, a.G - g0);
  const int head0 = kvh * a.G + g0;

  for (int e = tid; e < gc * D; e += kGenThreads) {
    const int g = e / D, d = e % D;
    float v = 0.f;
    if (g < ng) {
      v = Elem<DT>::to_f32(a.q[static_cast<int64_t>(tok) * a.q_st + static_cast<int64_t>(head0 + g) * a.q_sh + d]);
    }
    qs[e] = v * a.scale_log2;
    acc[e] = 0.f;
  }
  for (int g = tid; g < gc; g += kGenThreads) {
    mrun[g] = -1e30f;  // finite floor: 2^(m - m) = 1 and masked weights 2^(-inf - m) = 0
    lrun[g] = 0.f;
  }

  const int32_t* table = a.bt + static_cast<int64_t>(seq) * a.bt_sb;
  const int64_t hoff = static_cast<int64_t>(kvh) * a.c_sh;
  for (int t0 = 0; t0 < limit; t0 += kGenTile) {
    __syncthreads();  // the previous tile's weights and rows are consumed
    for (int e = tid; e < kGenTile * D; e += kGenThreads) {
      const int t = e / D, d = e % D;
      const int key = t0 + t;
      float kv = 0.f, vv = 0.f;
      if (key < limit) {
        int32_t page = table[key / a.bs];
        if (static_cast<uint32_t>(page) >= static_cast<uint32_t>(a.num_blocks)) page = 0;
        const int64_t off = static_cast<int64_t>(page) * a.c_sb + static_cast<int64_t>(key % a.bs) * a.c_st + hoff + d;
        kv = Elem<DT>::to_f32(a.kc[off]);
        vv = Elem<DT>::to_f32(a.vc[off]);
      }
      kt[e] = kv;
      vt[e] = vv;
    }
    __syncthreads();
    for (int e = tid; e < gc * kGenTile; e += kGenThreads) {
      const int g = e / kGenTile, t = e % kGenTile;
      float s = 0.f;
      for (int d = 0; d < D; ++d) s = fmaf(qs[g * D + d], kt[t * D + d], s);
      sc[e] = t0 + t < limit ? s : -INFINITY;
    }
    __syncthreads();
    for (int g = tid; g < gc; g += kGenThreads) {
      float mx = -INFINITY;
      for (int t = 0; t < kGenTile; ++t) mx = fmaxf(mx, sc[g * kGenTile + t]);
      const float m_new = fmaxf(mrun[g], mx);
      float sum = 0.f;
      for (int t = 0; t < kGenTile; ++t) {
        const float p = exp2f(sc[g * kGenTile + t] - m_new);
        sc[g * kGenTile + t] = p;
        sum += p;
      }
      const float al = exp2f(mrun[g] - m_new);
      alpha[g] = al;
      lrun[g] = lrun[g] * al + sum;
      mrun[g] = m_new;
    }
    __syncthreads();
    for (int e = tid; e < gc * D; e += kGenThreads) {
      const int g = e / D, d = e % D;
      float o = acc[e] * alpha[g];
      for (int t = 0; t < kGenTile; ++t) o = fmaf(sc[g * kGenTile + t], vt[t * D + d], o);
      acc[e] = o;
    }
  }
  __syncthreads();
  for (int e = tid; e < ng * D; e += kGenThreads) {
    const int g = e / D, d = e % D;
    const float l = lrun[g];
    const float o = l > 0.f ? acc[e] / l : 0.f;  // a row that sees no key gives 0
    a.out[static_cast<int64_t>(tok) * a.o_st + static_cast<int64_t>(head0 + g) * a.o_sh + d] = Elem<DT>::from_f32(o);
  }
}

// Heads per workgroup: the LDS holds q and O for gc heads (gc x D <=
// kGenMaxChunkElems) and their scores beside two tiles of K and V rows, at
// most 4 * (2 * 2048 + 2 * 16 * 256 + 64 * 16 + 3 * 64) bytes (~53 KB, under
// the 64 KB a launch gets without raising its limit).
static int general_chunk(int G, int D) {
  int gc = kGenMaxChunkElems / D;
  if (gc > kGenMaxHeads) gc = kGenMaxHeads;
  return G < gc ? G : gc;
}

static size_t general_lds_bytes(int gc, int D) {
  return static_cast<size_t>(4) * (2 * gc * D + 2 * kGenTile * D + gc * kGenTile + 3 * gc);
}

bool general_shape(int32_t head_dim, int32_t block_size) {
  return !(block_size == 16 && (head_dim == 64 || head_dim == 128));
}

int general_check(int32_t head_dim, int32_t block_size) {
  if (head_dim <= 0 || head_dim > kGenMaxHeadDim || block_size <= 0) return NIMBUS_ERR_UNSUPPORTED;
  return 0;
}

template <bool PREFILL>
static int launch_general(AttnGeneralArgs a, int64_t rows, int dtype, hipStream_t s) {
  a.gc = general_chunk(a.G, a.D);
  a.nchunks = (a.G + a.gc - 1) / a.gc;
  if (rows <= 0) return 0;
  if (rows > INT32_MAX || static_cast<int64_t>(a.KV) * a.nchunks > 65535) return NIMBUS_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(rows), a.KV * a.nchunks);
  const size_t lds = general_lds_bytes(a.gc, a.D);
  if (dtype == kFloat16) {
    hipLaunchKernelGGL((paged_general_kernel<kFloat16, PREFILL>), grid, dim3(kGenThreads), lds, s, a);
  } else {
    hipLaunchKernelGGL((paged_general_kernel<kBFloat16, PREFILL>), grid, dim3(kGenThreads), lds, s, a);
  }
  return static_cast<int>(hipGetLastError());
}

int launch_general_decode(const AttnGeneralArgs& a, int64_t batch, int dtype, hipStream_t s) {
  return launch_general<false>(a, batch * a.nq, dtype, s);
}

int launch_general_prefill(const AttnGeneralArgs& a, int64_t num_programs, int dtype, hipStream_t s) {
  return launch_general<true>(a, num_programs * a.tile_pos, dtype, s);
}

}  // namespace nimbus
