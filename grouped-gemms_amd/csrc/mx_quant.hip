// MX quantizer kernels: per-32-element FLOOR e8m0 scale + e4m3 / e2m1 cast.
//
// Row-wise kernel (`mxgg_quantize_mx`, the reference's `to_mx`, utils.py:67-105):
// four lanes own one 32-element block (8 elements each), so a wave reads 16
// consecutive blocks of a row with fully coalesced 16-byte loads (four such
// runs in flight), reduces the block amax with two lane shuffles, and writes 8
// e4m3 bytes (or 4 packed e2m1 bytes) per lane.  HBM-bound: 3.03 B/element
// for bf16 -> e4m3.
//
// Column-wise kernel (`mxgg_quantize_mx_dim0`, i.e. to_mx(x.t().contiguous())
// used for the weight-gradient operands, kernels/backward.py:232-243): a
// workgroup stages a 128 x 128 tile through LDS and each thread quantizes
// column blocks, so every line of the transposed output (128 source rows of
// one column) is written whole by one workgroup.
//
// Both-ways kernel (`mxgg_quantize_mx_both`): the same tile also yields the
// row-wise blocks, so one read of the source gives to_mx(x) and
// to_mx(x.t().contiguous()): 2 + 2 * (1 + 1/32) = 4.06 bytes per bf16
// element instead of 6.06 for the two passes.
//
// The e4m3 cast is the hardware fp8 conversion of the clamped, exactly
// scaled value (round to nearest even); blocks holding a NaN take the
// bit-level path, which keeps the NaN's sign as the reference's cast does.
//
// Scales go out in the reference's plain layout (row-major (rows, blocks)
// bytes) or step-major, the layout the GEMM kernels read (MXGG_SCALES_STEPS:
// for batches of R rows, dword (b, t, r) holds blocks 4t .. 4t+3 of row
// b*R + r, bytes past the row's last block 127), so a GEMM given them skips
// its per-call re-layout.
//
// E4M3 data goes out row-major or, on request (MXGG_DATA_PAIRS), in row
// pairs: byte k of row r at (r/2) 2 ld + (k/64) 128 + (r%2) 64 + k%64, the
// layout in which the GEMM's 64-element stage of two adjacent rows is one
// 128-byte line; packed E2M1 data (32 bytes per stage of a row) likewise in
// row quads (MXGG_DATA_QUADS): (r/4) 4 ld + (k/32) 128 + (r%4) 32 + k%32.
// Every store of these kernels (4, 8 or 32 bytes at a multiple of its size)
// stays inside one piece, so only the address changes; the pad of a row
// whose last piece is half full is written zero.
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

// Scale bytes of blocks blk0 .. blk0+n-1 of global row r (blk0 % 4 == 0,
// 1 <= n <= 4; byte j of w for block blk0 + j), from one lane: one dword
// store where the layout allows it.  n < 4 only where the row ends, so in the
// step-major layout the bytes past n are the neutral 127.
__device__ __forceinline__ void put_scale4(const ScaleOut& o, int64_t r, int64_t blk0, uint32_t w, int n) {
  if (o.steps) {
    if (n < 4) w = (w & ((1u << (8 * n)) - 1u)) | (0x7f7f7f7fu << (8 * n));
    const int64_t b = r / o.ld, rr = r - b * o.ld;
    *reinterpret_cast<uint32_t*>(o.p + ((b * o.T + (blk0 >> 2)) * o.ld + rr) * 4) = w;
    return;
  }
  uint8_t* d = o.p + r * o.ld + blk0;
  if (n == 4 && ((uintptr_t)d & 3) == 0) {
    *reinterpret_cast<uint32_t*>(d) = w;
    return;
  }
  for (int j = 0; j < n; ++j) d[j] = (uint8_t)(w >> (8 * j));
}

// The 4 scale bytes of a group of four consecutive lanes (lane j of the
// group holds block j's byte s), gathered into every lane of the group.
__device__ __forceinline__ uint32_t gather4(uint32_t s, int j) {
  uint32_t v = s << (8 * j);
  v |= (uint32_t)__shfl_xor((int)v, 1, 4);
  v |= (uint32_t)__shfl_xor((int)v, 2, 4);
  return v;
}

// Offset of byte k of row r of a quantizer output with row stride ld, in
// groups of 2**pl rows interleaved in 128 >> pl byte pieces (pl = 0: rows;
// 1: pairs; 2: quads; the store stays inside one piece).
__device__ __forceinline__ int64_t q_off(int64_t r, int64_t k, int64_t ld, int pl) {
  const int pb = 7 - pl;
  return (r >> pl) * (ld << pl) + ((k >> pb) << 7) + ((r & ((1 << pl) - 1)) << pb) + (k & ((1 << pb) - 1));
}

__device__ __forceinline__ void zero32(uint8_t* dst) {
  *reinterpret_cast<uint4*>(dst) = make_uint4(0, 0, 0, 0);
  *reinterpret_cast<uint4*>(dst + 16) = make_uint4(0, 0, 0, 0);
}

// 16 source bytes, read once: a non-temporal load, which leaves the lines
// already in L2 / the memory-side cache (often the producer's dirty output)
// in place instead of evicting them.  Streaming 16640 x 8192 bf16 after a
// 512 MB cache-dirtying fill: 98 us instead of 121 us for a copy-shaped
// kernel; with clean caches both take 82 us.
__device__ __forceinline__ uint4 load16_stream(const uint8_t* p) {
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <int SRC>
__device__ __forceinline__ void load8(const uint8_t* p, float (&v)[8]) {
  if constexpr (SRC == MXGG_DTYPE_BF16) {
    uint4 u = load16_stream(p);
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = bf16_to_f32(w[i] & 0xffffu);
      v[2 * i + 1] = bf16_to_f32(w[i] >> 16);
    }
  } else if constexpr (SRC == MXGG_DTYPE_F16) {
    uint4 u = load16_stream(p);
    const _Float16* h = reinterpret_cast<const _Float16*>(&u);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)h[i];
  } else {
    uint4 u0 = load16_stream(p);
    uint4 u1 = load16_stream(p + 16);
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

template <int SRC>
__device__ __forceinline__ float elem_to_f32(const uint8_t* p) {
  if constexpr (SRC == MXGG_DTYPE_BF16) return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
  else if constexpr (SRC == MXGG_DTYPE_F16) return (float)*reinterpret_cast<const _Float16*>(p);
  else return *reinterpret_cast<const float*>(p);
}

// e4m3 codes of a, b, c, d (bytes 0..3): clamp(x * mul, -448, 448) rounded
// to nearest even by the hardware fp8 conversion -- the bytes of the
// reference's clamp-then-cast (utils.py:97-102) for every input but NaN,
// which the caller routes to e4m3x4_sw.  mul is an exact power of two, inf
// clamps to +-448 like the reference's clamp, and a product that is an fp32
// subnormal rounds to a signed zero either way.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d, float mul) {
  const float ya = __builtin_amdgcn_fmed3f(a * mul, -448.f, 448.f);
  const float yb = __builtin_amdgcn_fmed3f(b * mul, -448.f, 448.f);
  const float yc = __builtin_amdgcn_fmed3f(c * mul, -448.f, 448.f);
  const float yd = __builtin_amdgcn_fmed3f(d * mul, -448.f, 448.f);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(ya, yb, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(yc, yd, (int)lo, true);
}

// The same four codes by the bit-level conversion (any input, NaN included:
// NaN keeps its sign, 0x7f / 0xff).
__device__ __forceinline__ uint32_t e4m3x4_sw(float a, float b, float c, float d, float mul) {
  return e4m3_code(a, mul) | (e4m3_code(b, mul) << 8) | (e4m3_code(c, mul) << 16) | (e4m3_code(d, mul) << 24);
}

// max |x| bit pattern of n fp32 values (NaN above inf, as the reference's amax
// propagates NaN).
template <int N>
__device__ __forceinline__ uint32_t amax_bits(const float* v) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const uint32_t a = abs_bits(v[i]);
    m = a > m ? a : m;
  }
  return m;
}

// One 32-element block held by one lane: FLOOR scale (returned), 32 e4m3
// bytes at dst (16-byte aligned).
__device__ __forceinline__ uint32_t quant32(const float (&v)[32], uint8_t* dst) {
  const uint32_t m = amax_bits<32>(v);
  const uint32_t sc = floor_scale(m, 8);
  const float mul = inv_scale(sc);
  uint32_t w[8];
  if (m > 0x7f800000u) {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = e4m3x4_sw(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3], mul);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = e4m3x4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3], mul);
  }
  *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
  *reinterpret_cast<uint4*>(dst + 16) = make_uint4(w[4], w[5], w[6], w[7]);
  return sc;
}

// Row-wise quantization: four lanes (a quad) own one 32-element block, 8
// elements each; a workgroup's 64 quads take 64 consecutive blocks (a
// contiguous 4 KB of bf16), one grid-stride pass per 64 * gridDim.x blocks.
// When rows hold a multiple of 4 blocks, four consecutive quads' scale bytes
// (one step of a row) go out as one dword.  I: the block index type (32-bit
// when the block count fits: one cheap division per block).  pl: output in
// row pairs (e4m3, pl = 1) or row quads (e2m1, pl = 2).
template <int SRC, int FMT, class I>
__global__ __launch_bounds__(256) void quant_rows_kernel(const uint8_t* __restrict__ src,
                                                         int64_t rows, int64_t cols,
                                                         int64_t ld_src_bytes,
                                                         uint8_t* __restrict__ q, int64_t ld_q, int pl,
                                                         ScaleOut so) {
  const I bpr = (I)(cols / 32);                        // blocks per row
  const I nblk = (I)rows * bpr;
  const int sub = threadIdx.x & 3;                     // which 8 of the 32
  const int qd = (threadIdx.x >> 2) & 3;               // quad within a group of four
  const bool by4 = bpr % 4 == 0;
  const I stride = (I)gridDim.x * 64;
  for (I base = (I)blockIdx.x * 64; base < nblk; base += stride) {
    // every lane of the wave runs each pass (the scale gathers are wave-wide);
    // lanes of blocks past nblk load and store nothing
    const I b = base + (I)(threadIdx.x >> 2);
    const bool live = b < nblk;
    const I r = live ? b / bpr : 0;
    const I cb = live ? b - r * bpr : 0;
    const int64_t col = (int64_t)cb * 32 + sub * 8;
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (live) load8<SRC>(src + (int64_t)r * ld_src_bytes + col * elem_bytes<SRC>(), v);
    uint32_t m = amax_bits<8>(v);
    const uint32_t m1 = (uint32_t)__shfl_xor((int)m, 1, 4);
    m = m1 > m ? m1 : m;
    const uint32_t m2 = (uint32_t)__shfl_xor((int)m, 2, 4);
    m = m2 > m ? m2 : m;
    const uint32_t s = floor_scale(m, FMT == MXGG_FMT_E4M3 ? 8 : 2);
    const float mul = inv_scale(s);
    if (live) {
      if constexpr (FMT == MXGG_FMT_E4M3) {
        uint32_t lo, hi;
        if (m > 0x7f800000u) {
          lo = e4m3x4_sw(v[0], v[1], v[2], v[3], mul);
          hi = e4m3x4_sw(v[4], v[5], v[6], v[7], mul);
        } else {
          lo = e4m3x4(v[0], v[1], v[2], v[3], mul);
          hi = e4m3x4(v[4], v[5], v[6], v[7], mul);
        }
        *reinterpret_cast<uint2*>(q + q_off(r, col, ld_q, pl)) = make_uint2(lo, hi);
        // row pairs, odd block count: the last block's lanes zero the pad
        if (pl && (bpr & 1) && cb == bpr - 1)
          *reinterpret_cast<uint2*>(q + q_off(r, col + 32, ld_q, pl)) = make_uint2(0, 0);
      } else {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) w |= e2m1_code(v[i], mul) << (4 * i);
        *reinterpret_cast<uint32_t*>(q + q_off(r, col / 2, ld_q, pl)) = w;
        // row quads, odd block count: the last block's lanes zero the pad
        if (pl && (bpr & 1) && cb == bpr - 1) *reinterpret_cast<uint32_t*>(q + q_off(r, col / 2 + 16, ld_q, pl)) = 0u;
      }
    }
    if (by4) {
      // quads 4k .. 4k+3 of a wave hold blocks 4k' .. 4k'+3 of one row (base
      // is a multiple of 64, rows a multiple of 4 blocks)
      uint32_t w4 = s << (8 * qd);
      w4 |= (uint32_t)__shfl_xor((int)w4, 4, 16);
      w4 |= (uint32_t)__shfl_xor((int)w4, 8, 16);
      if (live && qd == 0 && sub == 0) {
        const I left = nblk - b;
        put_scale4(so, r, cb, w4, left < 4 ? (int)left : 4);
      }
    } else if (live && sub == 0) {
      put_scale(so, r, cb, s);
    }
  }
}

// Column-wise quantization with transposed output (to_mx of the transpose),
// and with ROWS the row-wise quantization of the same data: one 128 x 128
// source tile per workgroup (batch blockIdx.z) staged through LDS.  Four
// consecutive lanes own the four 32-element blocks of one 128-element line of
// an output -- a column of the tile (source rows 32j .. 32j+31 in lane j) or a
// row of it (columns 32j .. 32j+31) -- so one store instruction writes whole
// 128-byte output lines and the group's four scale bytes leave as one dword.
// In LDS, 32-row band k of the tile is rotated by 16k columns, so the four
// lanes of a group, reading four bands of one column, hit disjoint banks.
// rows % 32 == 0: a partial last tile has whole 32-row blocks.  pl: outputs
// in row pairs (rows and cols even, so a batch is whole pairs).
template <int SRC, bool ROWS>
__global__ __launch_bounds__(256) void quant_tile_kernel(
    const uint8_t* __restrict__ src, int64_t rows, int64_t cols, int64_t ld_src_bytes, uint8_t* __restrict__ q_r,
    int64_t ld_qr, ScaleOut s_r, uint8_t* __restrict__ q_c, int64_t ld_qc, ScaleOut s_c, int pl) {
  constexpr int EB = elem_bytes<SRC>();
  constexpr int T = 128;                              // tile rows and columns
  constexpr int PITCH = T * EB + 16;                  // LDS row pitch, bytes
  constexpr int EPC = 16 / EB;                        // elements per 16-byte chunk
  constexpr int CPR = T / EPC;                        // chunks per tile row
  constexpr int NCH = T * CPR / 256;                  // chunks per thread
  __shared__ __attribute__((aligned(16))) uint8_t tile[T * PITCH];
  // byte offset of element (r, c) of the tile
  auto at = [](int r, int c) { return r * PITCH + (((c + 16 * (r >> 5)) & (T - 1)) * EB); };
  const int64_t b = blockIdx.z;
  src += b * rows * ld_src_bytes;
  q_c += b * cols * ld_qc;
  if constexpr (ROWS) q_r += b * rows * ld_qr;
  const int64_t r0 = (int64_t)blockIdx.y * T;
  const int64_t c0 = (int64_t)blockIdx.x * T;
  const int tr = (int)(rows - r0 < T ? rows - r0 : T);
  const int tc = (int)(cols - c0 < T ? cols - c0 : T);
  const int t = threadIdx.x;
  {
    uint4 u[NCH];
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int idx = t + 256 * i;
      const int rr = idx / CPR, c = (idx % CPR) * EPC;
      u[i] = (rr < tr && c < tc) ? load16_stream(src + (r0 + rr) * ld_src_bytes + (c0 + c) * EB)
                                 : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int idx = t + 256 * i;
      *reinterpret_cast<uint4*>(&tile[at(idx / CPR, (idx % CPR) * EPC)]) = u[i];
    }
  }
  __syncthreads();
  const int j = t & 3;                                // block of the lane within its line
  const int bands = tr / 32;                          // valid 32-row blocks of the tile
  // columns: group g = t / 4 + 64 pass owns tile column g (output row c0 + g)
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int c = t / 4 + 64 * pass;
    if (c < tc) {                                     // uniform over the four lanes
      uint32_t sc = 127;
      if (j < bands) {
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = elem_to_f32<SRC>(&tile[at(32 * j + i, c)]);
        sc = quant32(v, q_c + q_off(c0 + c, r0 + 32 * j, ld_qc, pl));
      } else if (pl && j == bands && (bands & 1)) {
        zero32(q_c + q_off(c0 + c, r0 + 32 * j, ld_qc, pl));   // pad of a row of 64k + 32 bytes
      }
      const uint32_t w4 = gather4(sc, j);
      if (j == 0) put_scale4(s_c, b * cols + c0 + c, r0 / 32, w4, bands < 4 ? bands : 4);
    }
  }
  if constexpr (ROWS) {
    // rows: group g = t / 4 + 64 pass owns tile row g (output row r0 + g)
    const int nb = tc / 32;                           // cols % 32 == 0
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
      const int r = t / 4 + 64 * pass;
      if (r < tr) {
        uint32_t sc = 127;
        if (j < nb) {
          float v[32];
#pragma unroll
          for (int k = 0; k < 32; k += EPC) {
            const uint4 ch = *reinterpret_cast<const uint4*>(&tile[at(r, 32 * j + k)]);
            const uint8_t* cp = reinterpret_cast<const uint8_t*>(&ch);
#pragma unroll
            for (int e = 0; e < EPC; ++e) v[k + e] = elem_to_f32<SRC>(cp + e * EB);
          }
          sc = quant32(v, q_r + q_off(r0 + r, c0 + 32 * j, ld_qr, pl));
        } else if (pl && j == nb && (nb & 1)) {
          zero32(q_r + q_off(r0 + r, c0 + 32 * j, ld_qr, pl));
        }
        const uint32_t w4 = gather4(sc, j);
        if (j == 0) put_scale4(s_r, b * rows + r0 + r, c0 / 32, w4, nb < 4 ? nb : 4);
      }
    }
  }
}

}  // namespace mxgg

using namespace mxgg;

namespace {

// Scale destination for `out_rows` rows of `nblk` blocks; MXGG_OK or a
// failure naming `what`.
int scale_out(const char* what, uint8_t* p, int64_t ld_s, int layout, int64_t out_rows, int64_t nblk, ScaleOut* o) {
  if (layout & ~(MXGG_SCALES_STEPS | MXGG_DATA_PAIRS | MXGG_DATA_QUADS) ||
      ((layout & MXGG_DATA_PAIRS) && (layout & MXGG_DATA_QUADS)))
    return fail(MXGG_ERR_INVALID_ARG, "%s: layout %d not PLAIN/STEPS, optionally | DATA_PAIRS or DATA_QUADS", what,
                layout);
  layout &= MXGG_SCALES_STEPS;
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

// A data output of `rows` rows of `len` bytes in groups of g rows (2: pairs,
// 4: quads) of 128 / g byte pieces: rows divisible by g, row stride a
// multiple of the piece that holds the row rounded up to it.
int pairs_out(const char* what, int64_t rows, int64_t len, int64_t ld, int g = 2) {
  const int64_t piece = 128 / g;
  if (rows % g)
    return fail(MXGG_ERR_INVALID_ARG, "%s: row %s need a row count divisible by %d, got %lld", what,
                g == 2 ? "pairs" : "quads", g, (long long)rows);
  if (ld % piece || ld < (len + piece - 1) / piece * piece)
    return fail(MXGG_ERR_INVALID_ARG, "%s: row %s need a row stride that is a multiple of %lld and holds %lld bytes",
                what, g == 2 ? "pairs" : "quads", (long long)piece, (long long)((len + piece - 1) / piece * piece));
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
  const int pl = (scale_layout & MXGG_DATA_PAIRS) ? 1 : ((scale_layout & MXGG_DATA_QUADS) ? 2 : 0);
  if ((pl == 1 && elem_fmt != MXGG_FMT_E4M3) || (pl == 2 && elem_fmt != MXGG_FMT_E2M1))
    return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx: row pairs hold e4m3 data and row quads packed e2m1");
  if (pl) {
    if (int rc = pairs_out("quantize_mx", rows, qcols, ld_q, 1 << pl)) return rc;
  }
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !q || !scales) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: null pointer");
  if (((uintptr_t)src % 16) || ((ld_src * eb) % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: source rows must be 16-byte aligned");
  if (elem_fmt == MXGG_FMT_E4M3 ? (((uintptr_t)q % 8) || (ld_q % 8)) : (((uintptr_t)q % 4) || (ld_q % 4)))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx: output rows misaligned");
  if (int rc = require_device()) return rc;
  const int64_t nblk = rows * (cols / 32);
  // 64 quads per 256-thread workgroup, one block each: one pass (the kernel
  // strides over the grid, so a capped grid only takes more passes)
  const int64_t want = (nblk + 63) / 64;
  const int grid = (int)(want < 1 ? 1 : (want < INT32_MAX ? want : INT32_MAX));
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s8 = (const uint8_t*)src;
  uint8_t* q8 = (uint8_t*)q;
  const int64_t lsb = ld_src * eb;
  const bool small = nblk + (int64_t)grid * 64 < ((int64_t)1 << 32);   // block indices fit 32 bits
#define MXGG_QROWS(SRC, FMT)                                                                               \
  do {                                                                                                     \
    if (small)                                                                                             \
      hipLaunchKernelGGL((quant_rows_kernel<SRC, FMT, uint32_t>), dim3(grid), dim3(256), 0, st, s8, rows,  \
                         cols, lsb, q8, ld_q, pl, so);                                                     \
    else                                                                                                   \
      hipLaunchKernelGGL((quant_rows_kernel<SRC, FMT, int64_t>), dim3(grid), dim3(256), 0, st, s8, rows,   \
                         cols, lsb, q8, ld_q, pl, so);                                                     \
  } while (0)
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
  if (scale_layout & MXGG_DATA_QUADS)
    return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_dim0: row quads hold packed e2m1 data; this output is e4m3");
  const int pl = (scale_layout & MXGG_DATA_PAIRS) ? 1 : 0;
  if (pl) {
    if (int rc = pairs_out("quantize_mx_dim0", cols, rows, ld_q)) return rc;
  }
  if (rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !q || !scales) return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: null pointer");
  if (((uintptr_t)src % 16) || ((ld_src * eb) % 16) || ((cols * eb) % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: source rows must be 16-byte aligned and a multiple of 16 bytes");
  if (((uintptr_t)q % 16) || (ld_q % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_dim0: output rows must be 16-byte aligned");
  if (int rc = require_device()) return rc;
  dim3 grid((unsigned)((cols + 127) / 128), (unsigned)((rows + 127) / 128));
  if (grid.y > 65535u) return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_dim0: too many rows");
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s8 = (const uint8_t*)src;
  const int64_t lsb = ld_src * eb;
  const ScaleOut none{};
#define MXGG_QCOLS(SRC) \
  hipLaunchKernelGGL((quant_tile_kernel<SRC, false>), grid, dim3(256), 0, st, s8, rows, cols, lsb, nullptr, 0, none, \
                     (uint8_t*)q, ld_q, so, pl)
  if (src_dtype == MXGG_DTYPE_BF16) MXGG_QCOLS(MXGG_DTYPE_BF16);
  else if (src_dtype == MXGG_DTYPE_F16) MXGG_QCOLS(MXGG_DTYPE_F16);
  else MXGG_QCOLS(MXGG_DTYPE_F32);
#undef MXGG_QCOLS
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
  if (scale_layout & MXGG_DATA_QUADS)
    return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_both: row quads hold packed e2m1 data; these outputs are e4m3");
  const int pl = (scale_layout & MXGG_DATA_PAIRS) ? 1 : 0;
  if (pl) {
    if (int rc = pairs_out("quantize_mx_both", rows, cols, ld_qr)) return rc;
    if (int rc = pairs_out("quantize_mx_both", cols, rows, ld_qc)) return rc;
  }
  if (batch == 0 || rows == 0 || cols == 0) return MXGG_OK;
  if (!src || !q_rows || !s_rows || !q_cols || !s_cols)
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: null pointer");
  const int eb = src_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  if (((uintptr_t)src % 16) || ((ld_src * eb) % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: source rows must be 16-byte aligned");
  if (((uintptr_t)q_rows % 16) || (ld_qr % 16) || ((uintptr_t)q_cols % 16) || (ld_qc % 16))
    return fail(MXGG_ERR_INVALID_ARG, "quantize_mx_both: output rows must be 16-byte aligned");
  if (int rc = require_device()) return rc;
  dim3 grid((unsigned)((cols + 127) / 128), (unsigned)((rows + 127) / 128), (unsigned)batch);
  if ((rows + 127) / 128 > 65535 || batch > 65535)
    return fail(MXGG_ERR_UNSUPPORTED, "quantize_mx_both: too many rows or batches");
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* s8 = (const uint8_t*)src;
  const int64_t lsb = ld_src * eb;
#define MXGG_QBOTH(SRC)                                                                                  \
  hipLaunchKernelGGL((quant_tile_kernel<SRC, true>), grid, dim3(256), 0, st, s8, rows, cols, lsb,         \
                     (uint8_t*)q_rows, ld_qr, sr, (uint8_t*)q_cols, ld_qc, sc, pl)
  if (src_dtype == MXGG_DTYPE_BF16) MXGG_QBOTH(MXGG_DTYPE_BF16);
  else if (src_dtype == MXGG_DTYPE_F16) MXGG_QBOTH(MXGG_DTYPE_F16);
  else MXGG_QBOTH(MXGG_DTYPE_F32);
#undef MXGG_QBOTH
  return launch_status("quantize_mx_both");
}
