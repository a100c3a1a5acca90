// MX quantizer kernels: per-32-element FLOOR e8m0 scale + e4m3 / e2m1 cast.
//
// Row-wise kernel (`mxgg_quantize_mx`, the reference's `to_mx`, utils.py:67-105):
// four lanes own one 32-element block (8 elements each), so a wave reads 16
// consecutive blocks of a row with fully coalesced 16-byte loads, reduces the
// block amax with two lane shuffles, and writes 8 e4m3 bytes (or 4 packed e2m1
// bytes) per lane.  HBM-bound: 3.03 B/element for bf16 -> e4m3.
//
// Column-wise kernel (`mxgg_quantize_mx_dim0`, i.e. to_mx(x.t().contiguous())
// used for the weight-gradient operands, kernels/backward.py:232-243): a
// workgroup stages a 32-row x 256-column tile through LDS and each thread
// quantizes one column block, writing the transposed row of the output.
//
// Both-ways kernel (`mxgg_quantize_mx_both`): the same tile also yields the
// row-wise blocks, so one read of the source gives to_mx(x) and
// to_mx(x.t().contiguous()): 2 + 2 * (1 + 1/32) = 4.06 bytes per bf16
// element instead of 6.06 for the two passes.
//
// Scales go out in the reference's plain layout (row-major (rows, blocks)
// bytes) or step-major, the layout the GEMM kernels read (MXGG_SCALES_STEPS:
// for batches of R rows, dword (b, t, r) holds blocks 4t .. 4t+3 of row
// b*R + r, bytes past the row's last block 127), so a GEMM given them skips
// its per-call re-layout.
#include "mxgg_device.h"
#include "mxgg_host.h"

namespace mxgg {

// Destination of a quantizer's scale bytes.  Row r counts over every batch.
struct ScaleOut {
  uint8_t* p;
  int64_t ld;       // plain: row stride; steps: R, rows per batch
  int64_t T;        // steps: dwords per row (cdiv(blocks, 4))
  int nblk;         // blocks per row
  bool steps;
};

__device__ __forceinline__ void put_scale(const ScaleOut& o, int64_t r, int64_t blk, uint32_t s) {
  if (!o.steps) {
    o.p[r * o.ld + blk] = (uint8_t)s;
    return;
  }
  const int64_t b = r / o.ld, rr = r - b * o.ld;
  uint8_t* d = o.p + ((b * o.T + (blk >> 2)) * o.ld + rr) * 4;
  const int j = (int)(blk & 3);
  d[j] = (uint8_t)s;
  if (blk == o.nblk - 1)                 // the last step's bytes past the row: neutral 2**0
    for (int k = j + 1; k < 4; ++k) d[k] = 127;
}

template <int SRC>
__device__ __forceinline__ void load8(const uint8_t* p, float (&v)[8]) {
  if constexpr (SRC == MXGG_DTYPE_BF16) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    }
  } else if constexpr (SRC == MXGG_DTYPE_F16) {
    uint4 u = *reinterpret_cast<const uint4*>(p);
    const _Float16* h = reinterpret_cast<const _Float16*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
  } else {
    uint4 u0 = *reinterpret_cast<const uint4*>(p);
    uint4 u1 = *reinterpret_cast<const uint4*>(p + 16);
    v[0] = __uint_as_float(u0.x); v[1] = __uint_as_float(u0.y);
    v[2] = __uint_as_float(u0.z); v[3] = __uint_as_float(u0.w);
    v[4] = __uint_as_float(u1.x); v[5] = __uint_as_float(u1.y);
    v[6] = __uint_as_float(u1.z); v[7] = __uint_as_float(u1.w);
  }
}

template <int SRC>
constexpr int elem_bytes() {
  return SRC == MXGG_DTYPE_F32 ? 4 : 2;
}

// One quad of lanes per block; grid-stride over all (row, block) pairs.
template <int SRC, int FMT>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint8_t* __restrict__ src,
                                                         int64_t rows, int64_t cols,
                                                         int64_t ld_src_bytes,
                                                         uint8_t* __restrict__ q, int64_t ld_q,
                                                         ScaleOut so) {
  const int64_t bpr = cols / 32;                       // blocks per row
  const int64_t nblk = rows * bpr;
  const int sub = threadIdx.x & 3;                     // which 8 of the 32
  const int64_t quads = (int64_t)gridDim.x * (blockDim.x / 4);
  for (int64_t b = (int64_t)blockIdx.x * (blockDim.x / 4) + (threadIdx.x >> 2); b < nblk + 0;
       b += quads) {
    // all four lanes of a quad share b, so the quad stays together in the loop
    const int64_t r = b / bpr;
    const int64_t cb = b - r * bpr;
    const int64_t col = cb * 32 + sub * 8;
    float v[8];
    load8<SRC>(src + r * ld_src_bytes + col * elem_bytes<SRC>(), v);
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t a = abs_bits(v[i]);
      m = a > m ? a : m;
    }
    uint32_t m1 = (uint32_t)__shfl_xor((int)m, 1, 4);
    m = m1 > m ? m1 : m;
    uint32_t m2 = (uint32_t)__shfl_xor((int)m, 2, 4);
    m = m2 > m ? m2 : m;
    const uint32_t s = floor_scale(m, FMT == MXGG_FMT_E4M3 ? 8 : 2);
    const float mul = inv_scale(s);
    if constexpr (FMT == MXGG_FMT_E4M3) {
      uint32_t lo = 0, hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) lo |= e4m3_code(v[i], mul) << (8 * i);
#pragma unroll
      for (int i = 0; i < 4; ++i) hi |= e4m3_code(v[4 + i], mul) << (8 * i);
      *reinterpret_cast<uint2*>(q + r * ld_q + col) = make_uint2(lo, hi);
    } else {
      uint32_t w = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) w |= e2m1_code(v[i], mul) << (4 * i);
      *reinterpret_cast<uint32_t*>(q + r * ld_q + col / 2) = w;
    }
    if (sub == 0) put_scale(so, r, cb, s);
  }
}

// Column-wise (dim-0) quantization with transposed output.  Tile: 32 source
// rows x 256 source columns per workgroup (256 threads, one column each).
template <int SRC>
__global__ __launch_bounds__(256) void quant_cols_kernel(const uint8_t* __restrict__ src,
                                                         int64_t rows, int64_t cols,
                                                         int64_t ld_src_bytes,
                                                         uint8_t* __restrict__ q, int64_t ld_q,
                                                         ScaleOut so) {
  constexpr int EB = elem_bytes<SRC>();
  constexpr int TC = 256;                         // tile columns
  __shared__ __attribute__((aligned(16))) uint8_t tile[32 * TC * EB];
  const int64_t r0 = (int64_t)blockIdx.y * 32;
  const int64_t c0 = (int64_t)blockIdx.x * TC;
  const int t = threadIdx.x;
  // cooperative 16-byte loads of the 32 x TC tile (columns past `cols` are
  // left untouched and never read back)
  constexpr int CHUNKS_PER_ROW = TC * EB / 16;
  for (int i = t; i < 32 * CHUNKS_PER_ROW; i += 256) {
    int rr = i / CHUNKS_PER_ROW;
    int cc = i - rr * CHUNKS_PER_ROW;
    int64_t col = c0 + (int64_t)cc * (16 / EB);
    if (col < cols) {
      uint4 u = *reinterpret_cast<const uint4*>(src + (r0 + rr) * ld_src_bytes + col * EB);
      *reinterpret_cast<uint4*>(&tile[(rr * TC) * EB + cc * 16]) = u;
    }
  }
  __syncthreads();
  const int64_t col = c0 + t;
  if (col >= cols) return;
  float v[32];
#pragma unroll
  for (int rr = 0; rr < 32; ++rr) {
    const uint8_t* p = &tile[(rr * TC + t) * EB];
    if constexpr (SRC == MXGG_DTYPE_BF16) {
      v[rr] = bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    } else if constexpr (SRC == MXGG_DTYPE_F16) {
      v[rr] = (float)*reinterpret_cast<const _Float16*>(p);
    } else {
      v[rr] = *reinterpret_cast<const float*>(p);
    }
  }
  uint32_t m = 0;
#pragma unroll
  for (int rr = 0; rr < 32; ++rr) {
    uint32_t a = abs_bits(v[rr]);
    m = a > m ? a : m;
  }
  const uint32_t s = floor_scale(m, 8);
  const float mul = inv_scale(s);
  uint32_t w[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w[i] = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[i] |= e4m3_code(v[4 * i + j], mul) << (8 * j);
  }
  uint8_t* dst = q + col * ld_q + r0;
  *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint4*>(dst + 16) = make_uint4(w[4], w[5], w[6], w[7]);
  put_scale(so, col, r0 / 32, s);
}

// Row-wise and column-wise quantization of one 32 x 256 tile of batch
// blockIdx.z: thread t quantizes the row block (row t / 8, columns
// 32 (t % 8) .. +31) and the column block (column t, the tile's 32 rows).
template <int SRC>
__global__ __launch_bounds__(256) void quant_both_kernel(const uint8_t* __restrict__ src,
                                                         int64_t rows, int64_t cols,
                                                         int64_t ld_src_bytes,
                                                         uint8_t* __restrict__ q_r, int64_t ld_qr, ScaleOut s_r,
                                                         uint8_t* __restrict__ q_c, int64_t ld_qc, ScaleOut s_c) {
  constexpr int EB = elem_bytes<SRC>();
  constexpr int TC = 256;
  __shared__ __attribute__((aligned(16))) uint8_t tile[32 * TC * EB];
  const int64_t b = blockIdx.z;
  src += b * rows * ld_src_bytes;
  q_r += b * rows * ld_qr;
  q_c += b * cols * ld_qc;
  const int64_t r0 = (int64_t)blockIdx.y * 32;
  const int64_t c0 = (int64_t)blockIdx.x * TC;
  const int t = threadIdx.x;
  constexpr int CHUNKS_PER_ROW = TC * EB / 16;
  for (int i = t; i < 32 * CHUNKS_PER_ROW; i += 256) {
    int rr = i / CHUNKS_PER_ROW;
    int cc = i - rr * CHUNKS_PER_ROW;
    int64_t col = c0 + (int64_t)cc * (16 / EB);
    if (col < cols) {
      uint4 u = *reinterpret_cast<const uint4*>(src + (r0 + rr) * ld_src_bytes + col * EB);
      *reinterpret_cast<uint4*>(&tile[(rr * TC) * EB + cc * 16]) = u;
    }
  }
  __syncthreads();
  auto load = [&](int rr, int cc) -> float {
    const uint8_t* p = &tile[(rr * TC + cc) * EB];
    if constexpr (SRC == MXGG_DTYPE_BF16) return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
    else if constexpr (SRC == MXGG_DTYPE_F16) return (float)*reinterpret_cast<const _Float16*>(p);
    else return *reinterpret_cast<const float*>(p);
  };
  // block blk of global row r (over every batch) of scale output so
  auto quant32 = [&](const float (&v)[32], uint8_t* dst, const ScaleOut& so, int64_t r, int64_t blk) {
    uint32_t m = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      uint32_t a = abs_bits(v[i]);
      m = a > m ? a : m;
    }
    const uint32_t sc = floor_scale(m, 8);
    const float mul = inv_scale(sc);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      w[i] = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) w[i] |= e4m3_code(v[4 * i + j], mul) << (8 * j);
    }
    *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    *reinterpret_cast<uint4*>(dst + 16) = make_uint4(w[4], w[5], w[6], w[7]);
    put_scale(so, r, blk, sc);
  };
  {
    const int rr = t / 8, cb = t % 8;
    const int64_t col0 = c0 + cb * 32;
    if (col0 < cols) {                             // cols % 32 == 0: whole blocks
      float v[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) v[i] = load(rr, cb * 32 + i);
      quant32(v, q_r + (r0 + rr) * ld_qr + col0, s_r, b * rows + r0 + rr, col0 / 32);
    }
  }
  {
    const int64_t col = c0 + t;
    if (col < cols) {
      float v[32];
#pragma unroll
      for (int rr = 0; rr < 32; ++rr) v[rr] = load(rr, t);
      quant32(v, q_c + col * ld_qc + r0, s_c, b * cols + col, r0 / 32);
    }
  }
}

}  // namespace mxgg

using namespace mxgg;

namespace {

// Scale destination for `out_rows` rows of `nblk` blocks; MXGG_OK or a
// failure naming `what`.
int scale_out(const char* what, uint8_t* p, int64_t ld_s, int layout, int64_t out_rows, int64_t nblk, ScaleOut* o) {
  if (layout != MXGG_SCALES_PLAIN && layout != MXGG_SCALES_STEPS)
    return fail(MXGG_ERR_INVALID_ARG, "%s: scale_layout %d not PLAIN/STEPS", what, layout);
  o->p = p;
  o->ld = ld_s;
  o->T = (nblk + 3) / 4;
  o->nblk = (int)nblk;
  o->steps = layout == MXGG_SCALES_STEPS;
  if (!o->steps) {
    if (ld_s < nblk) return fail(MXGG_ERR_INVALID_ARG, "%s: scale row stride smaller than the row", what);
  } else if (ld_s <= 0 || out_rows % ld_s) {
    return fail(MXGG_ERR_INVALID_ARG, "%s: step-major scales need ld_s = rows per batch, dividing the %lld rows", what,
                (long long)out_rows);
  }
  if (nblk > INT32_MAX) return fail(MXGG_ERR_UNSUPPORTED, "%s: rows too long", what);
  return MXGG_OK;
}

}  // namespace

extern "C" int mxgg_quantize_mx(const void* src, int src_dtype, int64_t rows, int64_t cols,
                                int64_t ld_src, int elem_fmt, void* q, int64_t ld_q,
                                uint8_t* scales, int64_t ld_s, int scale_layout, void* stream) {
  clear_error();
  if (src_dtype != MXGG_DTYPE_BF16 && src_dtype != MXGG_DTYPE_F16 && src_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: src_dtype %d not one of BF16/F16/F32", src_dtype);
  if (elem_fmt != MXGG_FMT_E4M3 && elem_fmt != MXGG_FMT_E2M1)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: elem_fmt %d not E4M3/E2M1", elem_fmt);
  if (rows < 0 || cols < 0) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: negative shape");
  if (cols % 32) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: last dim %lld must be divisible by block_size 32", (long long)cols);
  const int eb = src_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  const int64_t qcols = elem_fmt == MXGG_FMT_E4M3 ? cols : cols / 2;
  if (ld_src < cols || ld_q < qcols)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: row stride smaller than the row");
  ScaleOut so;
  if (int rc = scale_out("quantize_mx", scales, ld_s, scale_layout, rows, cols / 32, &so)) return rc;
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !q || !scales) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: null pointer");
  if (((uintptr_t)src % 16) || ((ld_src * eb) % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: source rows must be 16-byte aligned");
  if (elem_fmt == MXGG_FMT_E4M3 ? (((uintptr_t)q % 8) || (ld_q % 8)) : (((uintptr_t)q % 4) || (ld_q % 4)))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: output rows misaligned");
  if (int rc = require_device()) return rc;
  const int64_t nblk = rows * (cols / 32);
  int64_t want = (nblk + 63) / 64;                   // 64 blocks per 256-thread WG
  const int grid = (int)(want < 65536 ? (want < 1 ? 1 : want) : 65536);
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s8 = (const uint8_t*)src;
  uint8_t* q8 = (uint8_t*)q;
  const int64_t lsb = ld_src * eb;
#define MXGG_QROWS(SRC, FMT) \
  hipLaunchKernelGGL((quant_rows_kernel<SRC, FMT>), dim3(grid), dim3(256), 0, st, s8, rows, cols, lsb, q8, ld_q, so)
  if (elem_fmt == MXGG_FMT_E4M3) {
    if (src_dtype == MXGG_DTYPE_BF16) MXGG_QROWS(MXGG_DTYPE_BF16, MXGG_FMT_E4M3);
    else if (src_dtype == MXGG_DTYPE_F16) MXGG_QROWS(MXGG_DTYPE_F16, MXGG_FMT_E4M3);
    else MXGG_QROWS(MXGG_DTYPE_F32, MXGG_FMT_E4M3);
  } else {
    if (src_dtype == MXGG_DTYPE_BF16) MXGG_QROWS(MXGG_DTYPE_BF16, MXGG_FMT_E2M1);
    else if (src_dtype == MXGG_DTYPE_F16) MXGG_QROWS(MXGG_DTYPE_F16, MXGG_FMT_E2M1);
    else MXGG_QROWS(MXGG_DTYPE_F32, MXGG_FMT_E2M1);
  }
#undef MXGG_QROWS
  return launch_status("quantize_mx");
}

extern "C" int mxgg_quantize_mx_dim0(const void* src, int src_dtype, int64_t rows, int64_t cols,
                                     int64_t ld_src, int elem_fmt, void* q, int64_t ld_q,
                                     uint8_t* scales, int64_t ld_s, int scale_layout, void* stream) {
  clear_error();
  if (src_dtype != MXGG_DTYPE_BF16 && src_dtype != MXGG_DTYPE_F16 && src_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: src_dtype %d not one of BF16/F16/F32", src_dtype);
  if (elem_fmt != MXGG_FMT_E4M3)
    return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_dim0: only E4M3 output is built");
  if (rows < 0 || cols < 0) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: negative shape");
  if (rows % 32) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: dim 0 (%lld) must be divisible by block_size 32", (long long)rows);
  const int eb = src_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  if (ld_src < cols || ld_q < rows)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: row stride smaller than the row");
  ScaleOut so;
  if (int rc = scale_out("quantize_mx_dim0", scales, ld_s, scale_layout, cols, rows / 32, &so)) return rc;
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !q || !scales) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: null pointer");
  if (((uintptr_t)src % 16) || ((ld_src * eb) % 16) || ((cols * eb) % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: source rows must be 16-byte aligned and a multiple of 16 bytes");
  if (((uintptr_t)q % 16) || (ld_q % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: output rows must be 16-byte aligned");
  if (int rc = require_device()) return rc;
  dim3 grid((unsigned)((cols + 255) / 256), (unsigned)(rows / 32));
  if (grid.y > 65535u) return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_dim0: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s8 = (const uint8_t*)src;
  const int64_t lsb = ld_src * eb;
  if (src_dtype == MXGG_DTYPE_BF16)
    hipLaunchKernelGGL(quant_cols_kernel<MXGG_DTYPE_BF16>, grid, dim3(256), 0, st, s8, rows, cols, lsb, (uint8_t*)q, ld_q, so);
  else if (src_dtype == MXGG_DTYPE_F16)
    hipLaunchKernelGGL(quant_cols_kernel<MXGG_DTYPE_F16>, grid, dim3(256), 0, st, s8, rows, cols, lsb, (uint8_t*)q, ld_q, so);
  else
    hipLaunchKernelGGL(quant_cols_kernel<MXGG_DTYPE_F32>, grid, dim3(256), 0, st, s8, rows, cols, lsb, (uint8_t*)q, ld_q, so);
  return launch_status("quantize_mx_dim0");
}

extern "C" int mxgg_quantize_mx_both(const void* src, int src_dtype, int64_t batch, int64_t rows, int64_t cols,
                                     int64_t ld_src, void* q_rows, int64_t ld_qr, uint8_t* s_rows,
                                     int64_t ld_sr, void* q_cols, int64_t ld_qc, uint8_t* s_cols,
                                     int64_t ld_sc, int scale_layout, void* stream) {
  clear_error();
  if (src_dtype != MXGG_DTYPE_BF16 && src_dtype != MXGG_DTYPE_F16 && src_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: src_dtype %d not one of BF16/F16/F32", src_dtype);
  if (batch < 0 || rows < 0 || cols < 0) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: negative shape");
  if (rows % 32 || cols % 32)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: both dims (%lld, %lld) must be divisible by block_size 32",
                (long long)rows, (long long)cols);
  if (ld_src < cols || ld_qr < cols || ld_qc < rows)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: row stride smaller than the row");
  ScaleOut sr, sc;
  if (int rc = scale_out("quantize_mx_both", s_rows, ld_sr, scale_layout, batch * rows, cols / 32, &sr)) return rc;
  if (int rc = scale_out("quantize_mx_both", s_cols, ld_sc, scale_layout, batch * cols, rows / 32, &sc)) return rc;
  if (batch == 0 || rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !q_rows || !s_rows || !q_cols || !s_cols)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: null pointer");
  const int eb = src_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  if (((uintptr_t)src % 16) || ((ld_src * eb) % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: source rows must be 16-byte aligned");
  if (((uintptr_t)q_rows % 16) || (ld_qr % 16) || ((uintptr_t)q_cols % 16) || (ld_qc % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: output rows must be 16-byte aligned");
  if (int rc = require_device()) return rc;
  dim3 grid((unsigned)((cols + 255) / 256), (unsigned)(rows / 32), (unsigned)batch);
  if (rows / 32 > 65535 || batch > 65535) return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_both: too many rows or batches");
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s8 = (const uint8_t*)src;
  const int64_t lsb = ld_src * eb;
#define MXGG_QBOTH(SRC)                                                                                  \
  hipLaunchKernelGGL(quant_both_kernel<SRC>, grid, dim3(256), 0, st, s8, rows, cols, lsb, (uint8_t*)q_rows, \
                     ld_qr, sr, (uint8_t*)q_cols, ld_qc, sc)
  if (src_dtype == MXGG_DTYPE_BF16) MXGG_QBOTH(MXGG_DTYPE_BF16);
  else if (src_dtype == MXGG_DTYPE_F16) MXGG_QBOTH(MXGG_DTYPE_F16);
  else MXGG_QBOTH(MXGG_DTYPE_F32);
#undef MXGG_QBOTH
  return launch_status("quantize_mx_both");
}
