// Device-side helpers shared by the MX quantizer and the grouped-GEMM kernels
// (gfx950 / CDNA4 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxgg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kWave = 64;

// Wave index inside the workgroup, as a scalar (SGPR) value.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }


// ---------------------------------------------------------------------------
// element conversions (bit-exact with the FLOOR-mode `to_mx`, utils.py:84-105)
// ---------------------------------------------------------------------------

// |x| bits with NaN-propagating max semantics: as unsigned integers every NaN
// pattern (> 0x7f800000) compares above inf and every finite magnitude, and the
// scale depends only on the exponent field, which is 0xff for any NaN or inf.
__device__ __forceinline__ uint32_t abs_bits(float x) {
  return __float_as_uint(x) & 0x7fffffffu;
}

// FLOOR e8m0 scale from the max |x| bit pattern of a block:
// clamp(exponent(max(amax, fp32 tiny)) - max_pow2, 0, 254).
__device__ __forceinline__ uint32_t floor_scale(uint32_t amax_bits, int max_pow2) {
  uint32_t a = amax_bits < 0x00800000u ? 0x00800000u : amax_bits;
  int e = (int)(a >> 23);
  int s = e - max_pow2;
  s = s < 0 ? 0 : (s > 254 ? 254 : s);
  return (uint32_t)s;
}

// 2**(127 - s) as an fp32 (exact; 127-s stays inside the normal range for the
// scales floor_scale can return).
__device__ __forceinline__ float inv_scale(uint32_t s) {
  return __uint_as_float((254u - s) << 23);
}

// Round-half-even of mant / 2**shift for shift in [1, 31].
__device__ __forceinline__ uint32_t rne_shift(uint32_t mant, uint32_t shift) {
  uint32_t q = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1u);
  return q + ((rem > half) || (rem == half && (q & 1u)) ? 1u : 0u);
}

// fp32 -> e4m3fn code of clamp(v, -448, 448) with round-half-even; NaN keeps
// its sign bit and becomes the NaN code (0x7f / 0xff).
__device__ __forceinline__ uint32_t e4m3_from_scaled(float v) {
  uint32_t b = __float_as_uint(v);
  uint32_t sign = (b >> 24) & 0x80u;
  uint32_t a = b & 0x7fffffffu;
  uint32_t code;
  if (a > 0x7f800000u) {
    code = 0x7fu;                                    // NaN
  } else if (a >= 0x43e00000u) {
    code = 0x7eu;                                    // >= 448 (and inf): clamp
  } else if (a >= 0x3c800000u) {                     // >= 2**-6: normal e4m3
    uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);     // RNE at mantissa bit 20
    code = (r >> 20) - (120u << 3);                   // rebias 127 -> 7
  } else {                                           // subnormal grid, step 2**-9
    uint32_t e = a >> 23;
    uint32_t shift = 141u - e;                        // value*2**9 = mant / 2**shift
    code = (e == 0u || shift > 24u) ? 0u : rne_shift((a & 0x7fffffu) | 0x800000u, shift);
  }
  return code | sign;
}

// fp32 -> e2m1 nibble of clamp(v, -6, 6), round-half-even; NaN saturates to
// the max-magnitude code with its sign.
__device__ __forceinline__ uint32_t e2m1_from_scaled(float v) {
  uint32_t b = __float_as_uint(v);
  uint32_t sign = (b >> 28) & 0x8u;
  uint32_t a = b & 0x7fffffffu;
  uint32_t code;
  if (a >= 0x40c00000u) {
    code = 7u;                                       // >= 6, inf, NaN
  } else if (a >= 0x3f800000u) {                     // >= 1: one mantissa bit
    uint32_t r = a + 0x1fffffu + ((a >> 22) & 1u);
    code = (r >> 22) - (126u << 1);
  } else {                                           // [0, 1): step 0.5
    uint32_t e = a >> 23;
    uint32_t shift = 149u - e;
    code = (e == 0u || shift > 24u) ? 0u : rne_shift((a & 0x7fffffu) | 0x800000u, shift);
  }
  return code | sign;
}

// Element codes of x / 2**(s-127), computed as the exact product x * 2**(127-s).
// A NaN keeps the sign of the input NaN (not whatever sign the multiply gives).
__device__ __forceinline__ uint32_t e4m3_code(float x, float mul) {
  uint32_t c = e4m3_from_scaled(x * mul);
  uint32_t b = __float_as_uint(x);
  return (b & 0x7fffffffu) > 0x7f800000u ? (0x7fu | ((b >> 24) & 0x80u)) : c;
}

__device__ __forceinline__ uint32_t e2m1_code(float x, float mul) {
  uint32_t c = e2m1_from_scaled(x * mul);
  uint32_t b = __float_as_uint(x);
  return (b & 0x7fffffffu) > 0x7f800000u ? (0x7u | ((b >> 28) & 0x8u)) : c;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// fp32 -> bf16 bits, round-half-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  bf2 r;
  r[0] = (__bf16)lo;
  r[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(pack_bf16x2(x, 0.f) << 16);
}

// ---------------------------------------------------------------------------
// buffer resources (raw buffers: loads past num_records return zero)
// ---------------------------------------------------------------------------

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

constexpr uint32_t kOOB = 0x80000000u;  // voffset that is always out of range

// ---------------------------------------------------------------------------
// wave-level scans
// ---------------------------------------------------------------------------

// Inclusive prefix sum over the 64 lanes of a wave in DPP steps (no LDS):
// Hillis-Steele shifts by 1, 2, 4, 8 inside each 16-lane row, then the last
// lane of rows 0 and 2 is added to rows 1 and 3 (row_bcast:15) and lane 31 to
// rows 2 and 3 (row_bcast:31).  Sources outside the row, and rows the mask
// leaves out, contribute the `old` operand, 0.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);   // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);   // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);   // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);   // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15 into rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);   // row_bcast:31 into rows 2, 3
  return v;
}

// Value of v in lane `src` (wave-uniform src), as a scalar.
__device__ __forceinline__ int lane_value(int v, int src) { return __builtin_amdgcn_readlane(v, src); }

// ---------------------------------------------------------------------------
// routing (kernels/forward.py:296-365 semantics)
// ---------------------------------------------------------------------------

// Total number of BM-row tiles over all groups: sum_e cdiv(hist[e], BM), with
// hist[e] = offs[e] - offs[e-1] (negative treated as empty).  Every lane of the
// calling wave returns the same value.
__device__ __forceinline__ int route_total(const int32_t* __restrict__ offs, int E, int BM) {
  const int lane = threadIdx.x & (kWave - 1);
  int carry = 0;
  for (int base = 0; base < E; base += kWave) {
    int e = base + lane;
    int nb = 0;
    if (e < E) {
      int end = offs[e];
      int prev = e > 0 ? offs[e - 1] : 0;
      int h = end - prev;
      nb = h > 0 ? (h + BM - 1) / BM : 0;
    }
    int incl = wave_incl_scan(nb);
    carry += lane_value(incl, kWave - 1);
  }
  return carry;
}

struct TileRoute {
  int expert;    // group index
  int block;     // BM-row block inside the group
  int start;     // first row of the group (offs[e-1])
  int rows;      // valid rows of this tile (<= BM)
};

// Expert-aligned tile order used by the GEMMs: the tiles of group e (its
// cdiv(hist[e], BM) m-blocks x grid_n column tiles) are contiguous in the
// logical order, groups in order; inside a group the m-blocks form bands of
// at most group_m (balanced: nbands = cdiv(blocks, group_m), height
// cdiv(blocks, nbands), the last band shorter), column-major inside a band.
// Unlike the reference's GROUP_M bands over the global m-block index
// (kernels/forward.py:38-51), no band mixes two groups, so
// the tiles in flight on an XCD read one group's weights.  Returns the owner
// of logical tile t (0 <= t < total blocks x grid_n) and its column tile pn;
// expert < 0 past the end.  Wave-uniform.
// One 64-group chunk of the lookup: lane l holds group base + l (first row
// prev, rows h, blocks nb) and incl, the inclusive scan of nb over all groups
// up to it.  True, with r and pn filled, when a lane of the chunk owns t.
__device__ __forceinline__ bool route_tile_chunk(int base, int E, int BM, int grid_n, int group_m, int t,
                                                 int prev, int h, int nb, int incl, TileRoute& r, int& pn) {
  const int e = base + (int)(threadIdx.x & (kWave - 1));
  const int nt = nb * grid_n;
  const int tincl = incl * grid_n;
  const int texcl = tincl - nt;
  const bool own = (e < E) && (nt > 0) && (t >= texcl) && (t < tincl);
  const unsigned long long m = __ballot(own);
  if (!m) return false;
  const int src = __ffsll((long long)m) - 1;
  const int local = t - lane_value(texcl, src);
  const int blocks = lane_value(nb, src);
  const int hh = lane_value(h, src);
  const int g = group_m > 0 ? group_m : 1;
  const int nbands = (blocks + g - 1) / g;
  const int bh = (blocks + nbands - 1) / nbands;           // band height
  int b = local / (bh * grid_n);
  if (b > nbands - 1) b = nbands - 1;
  const int in_band = local - b * bh * grid_n;
  const int hb = b == nbands - 1 ? blocks - b * bh : bh;   // this band's height
  const int col = in_band / hb;
  r.expert = uniform(base + src);
  r.block = b * bh + (in_band - col * hb);
  r.start = lane_value(prev, src);
  const int rem = hh - r.block * BM;
  r.rows = rem < BM ? rem : BM;
  pn = col;
  return true;
}

__device__ __forceinline__ TileRoute route_tile(const int32_t* __restrict__ offs, int E, int BM, int grid_n,
                                                int group_m, int t, int& pn) {
  const int lane = threadIdx.x & (kWave - 1);
  TileRoute r{-1, 0, 0, 0};
  pn = 0;
  int carry = 0;
  for (int base = 0; base < E; base += kWave) {
    int e = base + lane;
    int nb = 0, h = 0, prev = 0;
    if (e < E) {
      int end = offs[e];
      prev = e > 0 ? offs[e - 1] : 0;
      h = end - prev;
      nb = h > 0 ? (h + BM - 1) / BM : 0;
    }
    const int incl = wave_incl_scan(nb) + carry;
    if (route_tile_chunk(base, E, BM, grid_n, group_m, t, prev, h, nb, incl, r, pn)) return r;
    carry = lane_value(incl, kWave - 1);
  }
  return r;
}

// Groups 0 .. E-1 of a launch with E <= 64, one per lane, read from offs once
// for both the block count (total) and the tile lookup (route_tile below).
struct WaveGroups {
  int prev, h, nb, incl;   // lane e: first row, rows, BM-row blocks, inclusive block scan
  int total;               // blocks over all groups (wave-uniform)
};

__device__ __forceinline__ WaveGroups load_groups(const int32_t* __restrict__ offs, int E, int BM) {
  const int e = threadIdx.x & (kWave - 1);
  WaveGroups g{0, 0, 0, 0, 0};
  if (e < E) {
    const int end = offs[e];
    g.prev = e > 0 ? offs[e - 1] : 0;
    g.h = end - g.prev;
    g.nb = g.h > 0 ? (g.h + BM - 1) / BM : 0;
  }
  g.incl = wave_incl_scan(g.nb);
  g.total = lane_value(g.incl, kWave - 1);
  return g;
}

__device__ __forceinline__ TileRoute route_tile(const WaveGroups& wg, int E, int BM, int grid_n, int group_m,
                                                int t, int& pn) {
  TileRoute r{-1, 0, 0, 0};
  pn = 0;
  route_tile_chunk(0, E, BM, grid_n, group_m, t, wg.prev, wg.h, wg.nb, wg.incl, r, pn);
  return r;
}

// XCD swizzle (kernels/forward.py:31-36): program ids are dispatched round-robin
// to X XCDs; give every XCD a contiguous range of the logical tile order.
__device__ __forceinline__ int xcd_swizzle(int pid, int domain, int X) {
  const int per = domain / X;
  const int extra = domain - per * X;
  const int q = pid / X;
  const int g = pid - q * X;
  return g * per + (g < extra ? g : extra) + q;
}

}  // namespace mxgg
