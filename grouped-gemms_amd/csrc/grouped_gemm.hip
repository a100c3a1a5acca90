// MX-scaled grouped GEMM kernels for gfx950 (CDNA4):
//   * forward / dgrad:  out[s:e] = A[s:e] @ B[g]^T          (kernels/forward.py:81-294)
//   * weight gradient:  out[g]   = GO[:, s:e] @ IA[:, s:e]^T (kernels/backward.py:31-215)
//   * routing table and tile schedule exposed for testing   (kernels/forward.py:31-51, 296-365)
//
// Both GEMMs are "NT" products whose two operands are contiguous along the
// reduction dimension, so they share one main loop:
//   acc[r][c] = sum_k X[r][k] * W[c][k] * 2**(xs[r][k/32]-127) * 2**(ws[c][k/32]-127)
// with X on the B side and W on the A side of v_mfma_scale_f32_32x32x64_f8f6f4,
// so that every lane of the accumulator holds 4 consecutive output columns.
//
// Main loop per 128-element reduction step (BK = 128):
//   * X and W tiles go global -> LDS directly with 16-byte buffer_load ... lds
//     (no VGPR staging); rows past the valid range and masked reduction chunks
//     read as zero through the buffer range check.
//   * LDS rows are 128 bytes (e4m3) or 64 bytes (packed e2m1) with 16-byte
//     chunks XOR-swizzled by row so the 32-row fragment reads are free of bank
//     conflicts for both 8- and 16-lane LDS service groups.
//   * two LDS stages (double buffering) and a software-pipelined loop with
//     one workgroup barrier per step (mainloop_pipe below).
//   * e8m0 scales are read straight from the plain `to_mx` layout: one dword
//     per tile row and step (the 4 scale bytes of the step's 4 32-element
//     blocks) travels global -> LDS next to the data, and each MFMA selects
//     its byte with op_sel.  Scale rows that are not 4-byte aligned take a
//     byte-gather register path (mainloop below).
#include "mxgg_device.h"
#include "mxgg_host.h"

namespace mxgg {

constexpr int BK = 128;

template <int BM_, int BN_, int WGM_, int WGN_, int WFMT_>
struct Cfg {
  static constexpr int BM = BM_;        // X rows per tile (output rows)
  static constexpr int BN = BN_;        // W rows per tile (output columns)
  static constexpr int WGM = WGM_;      // waves along rows
  static constexpr int WGN = WGN_;      // waves along columns
  static constexpr int WFMT = WFMT_;    // W element format (X is always e4m3)
  static constexpr int NW = WGM * WGN;
  static constexpr int NT = NW * kWave;
  static constexpr int WTM = BM / WGM;
  static constexpr int WTN = BN / WGN;
  static constexpr int FM = WTM / 32;
  static constexpr int FN = WTN / 32;
  static constexpr int XROW = BK;                                  // bytes per X row per step
  static constexpr int WROW = WFMT == MXGG_FMT_E2M1 ? BK / 2 : BK;  // bytes per W row per step
  static constexpr int XBYTES = BM * XROW;
  static constexpr int WBYTES = BN * WROW;
  static constexpr int XSOFF = XBYTES + WBYTES;                   // X scale dwords (BM x 4 B)
  static constexpr int WSOFF = XSOFF + BM * 4;                     // W scale dwords (BN x 4 B)
  static constexpr int STAGE = WSOFF + BN * 4;
  static constexpr int QX = XBYTES / 1024 / NW;                   // 1 KB loads per wave
  static constexpr int QW = WBYTES / 1024 / NW;
  static constexpr int QS = (BM + BN) / 64 / NW;                   // 256 B scale loads per wave
  static_assert(XBYTES % (1024 * NW) == 0 && WBYTES % (1024 * NW) == 0, "tile/wave split");
  static_assert((BM + BN) % (64 * NW) == 0 && BM % 64 == 0, "scale/wave split");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
};

// 16-byte chunk swizzles (see header comment): bijective on the chunk index for
// every 8-row and every parity class of 16 rows (128-byte rows), resp. every
// 4-row class of 8 and 16 rows (64-byte rows).
__device__ __forceinline__ int swz8(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
__device__ __forceinline__ int swz4(int r) {
  return ((((r >> 2) ^ (r >> 3)) & 1) << 1) | (((r >> 1) ^ (r >> 2)) & 1);
}

struct Operand {
  __amdgpu_buffer_rsrc_t data;   // base = first row of the tile; range = valid rows
  __amdgpu_buffer_rsrc_t scale;  // base = scales of the first row; range = valid rows
  uint32_t ld;                   // bytes between rows
  uint32_t lds;                  // scale bytes between rows
};

template <class C>
struct LoadPlan {
  uint32_t xoff[C::QX];     // per-lane byte offset of each 1 KB X load (row * ld + chunk)
  uint32_t woff[C::QW];
  int xk[C::QX];            // reduction element of the lane's X chunk inside the step
  int wk[C::QW];
  uint32_t xs_off[C::FM];   // per-lane scale row offsets (register path)
  uint32_t ws_off[C::FN];
  uint32_t s_off[C::QS];    // per-lane scale row offsets (LDS path, one row per lane)
};

template <class C>
__device__ __forceinline__ void make_plan(LoadPlan<C>& P, const Operand& X, const Operand& W) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int i = 0; i < C::QX; ++i) {
    int q = wave * C::QX + i;
    int row = q * 8 + lane / 8;
    int c = (lane & 7) ^ swz8(row);
    P.xoff[i] = (uint32_t)row * X.ld + (uint32_t)c * 16u;
    P.xk[i] = c * 16;
  }
#pragma unroll
  for (int i = 0; i < C::QW; ++i) {
    int q = wave * C::QW + i;
    if constexpr (C::WFMT == MXGG_FMT_E2M1) {
      int row = q * 16 + lane / 4;
      int c = (lane & 3) ^ swz4(row);
      P.woff[i] = (uint32_t)row * W.ld + (uint32_t)c * 16u;
      P.wk[i] = c * 32;
    } else {
      int row = q * 8 + lane / 8;
      int c = (lane & 7) ^ swz8(row);
      P.woff[i] = (uint32_t)row * W.ld + (uint32_t)c * 16u;
      P.wk[i] = c * 16;
    }
  }
  const int wm = wave / C::WGN, wn = wave % C::WGN;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) P.xs_off[i] = (uint32_t)(wm * C::WTM + i * 32 + lane % 32) * X.lds;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) P.ws_off[j] = (uint32_t)(wn * C::WTN + j * 32 + lane % 32) * W.lds;
#pragma unroll
  for (int i = 0; i < C::QS; ++i) {
    int row = (wave * C::QS + i) * 64 + lane;     // scale rows: X rows then W rows
    P.s_off[i] = row < C::BM ? (uint32_t)row * X.lds : (uint32_t)(row - C::BM) * W.lds;
  }
}

// LDS path: the step's scale dword of every X and W row of the tile, one row
// per lane, copied global -> LDS next to the data tiles.
template <class C>
__device__ __forceinline__ void issue_scales(uint8_t* sb, const Operand& X, const Operand& W,
                                             const LoadPlan<C>& P, int st) {
  const int wave = wave_id();
#pragma unroll
  for (int i = 0; i < C::QS; ++i) {
    const int q = wave * C::QS + i;               // 64-row group; uniform per wave
    const bool isx = q * 64 < C::BM;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(isx ? X.scale : W.scale,
                                             (lds_ptr_t)(sb + C::XSOFF + q * 256), 4, P.s_off[i],
                                             (uint32_t)st * 4u, 0, 0);
  }
}

// Issue the global->LDS copies of reduction step `st` into stage buffer `sb`.
// MASKED: chunks whose reduction range falls outside [lo, hi) load zeros.
template <class C, bool MASKED>
__device__ __forceinline__ void issue_tiles(uint8_t* sb, const Operand& X, const Operand& W,
                                            const LoadPlan<C>& P, int st, int lo, int hi) {
  const int wave = wave_id();
  const uint32_t xso = (uint32_t)st * C::XROW;
  const uint32_t wso = (uint32_t)st * C::WROW;
#pragma unroll
  for (int i = 0; i < C::QX; ++i) {
    uint32_t off = P.xoff[i];
    if constexpr (MASKED) {
      int k = st * BK + P.xk[i];
      if (k < lo || k + 16 > hi) off = kOOB;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(X.data, (lds_ptr_t)(sb + (wave * C::QX + i) * 1024), 16,
                                             off, xso, 0, 0);
  }
  uint8_t* wb = sb + C::XBYTES;
#pragma unroll
  for (int i = 0; i < C::QW; ++i) {
    uint32_t off = P.woff[i];
    if constexpr (MASKED) {
      int k = st * BK + P.wk[i];
      int w = C::WFMT == MXGG_FMT_E2M1 ? 32 : 16;
      if (k < lo || k + w > hi) off = kOOB;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(W.data, (lds_ptr_t)(wb + (wave * C::QW + i) * 1024), 16,
                                             off, wso, 0, 0);
  }
}

// Branch-free variant used by the pipelined loop: every load is range-checked
// with a select, so a step outside [lo, hi) (e.g. a prefetch past the last
// step) only writes zeros into the stage.
template <class C>
__device__ __forceinline__ void issue_tiles_sel(uint8_t* sb, const Operand& X, const Operand& W,
                                                const LoadPlan<C>& P, int st, int lo, int hi) {
  const int wave = wave_id();
  const uint32_t xso = (uint32_t)st * C::XROW;
  const uint32_t wso = (uint32_t)st * C::WROW;
  const int kk = st * BK;
  constexpr int WCH = C::WFMT == MXGG_FMT_E2M1 ? 32 : 16;
#pragma unroll
  for (int i = 0; i < C::QX; ++i) {
    const int k = kk + P.xk[i];
    const uint32_t off = (k >= lo && k + 16 <= hi) ? P.xoff[i] : kOOB;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(X.data, (lds_ptr_t)(sb + (wave * C::QX + i) * 1024), 16,
                                             off, xso, 0, 0);
  }
  uint8_t* wb = sb + C::XBYTES;
#pragma unroll
  for (int i = 0; i < C::QW; ++i) {
    const int k = kk + P.wk[i];
    const uint32_t off = (k >= lo && k + WCH <= hi) ? P.woff[i] : kOOB;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(W.data, (lds_ptr_t)(wb + (wave * C::QW + i) * 1024), 16,
                                             off, wso, 0, 0);
  }
}

// Byte mask (0xff per 32-element block) of the step's blocks outside [lo, hi).
__device__ __forceinline__ uint32_t outside_mask(int st, int lo, int hi) {
  uint32_t m = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const int k = st * BK + 32 * b;
    m |= (k < lo || k >= hi) ? (0xffu << (8 * b)) : 0u;
  }
  return m;
}

// Scale dwords of step `st`: byte b = scale of the 32-element block 4*st + b.
template <bool DW>
__device__ __forceinline__ uint32_t load_scale4(__amdgpu_buffer_rsrc_t r, uint32_t off, int st) {
  if constexpr (DW) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, (uint32_t)st * 4u, 0);
  } else {
    uint32_t v = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b)
      v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(r, off + b, (uint32_t)st * 4u, 0) << (8 * b);
    return v;
  }
}

// Replace the scale bytes of 32-element blocks outside [lo, hi) by 127 (2**0)
// so that masked (zero) data never meets a NaN scale byte.
__device__ __forceinline__ uint32_t neutralize(uint32_t v, int st, int lo, int hi) {
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    int k = st * BK + 32 * b;
    if (k < lo || k >= hi) v = (v & ~(0xffu << (8 * b))) | (127u << (8 * b));
  }
  return v;
}

template <class C, bool DW>
__device__ __forceinline__ void load_scales(uint32_t (&xs)[C::FM], uint32_t (&ws)[C::FN],
                                            const Operand& X, const Operand& W,
                                            const LoadPlan<C>& P, int st) {
#pragma unroll
  for (int i = 0; i < C::FM; ++i) xs[i] = load_scale4<DW>(X.scale, P.xs_off[i], st);
#pragma unroll
  for (int j = 0; j < C::FN; ++j) ws[j] = load_scale4<DW>(W.scale, P.ws_off[j], st);
}

// One 64-element half of a step: fragments from LDS, FM x FN scaled MFMAs.
template <class C, int H>
__device__ __forceinline__ void mma_half(const uint8_t* sb, const uint32_t (&xs)[C::FM],
                                         const uint32_t (&ws)[C::FN],
                                         v16f (&acc)[C::FM][C::FN]) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int hsel = lane >> 5;
  const int r32 = lane & 31;
  const int sw8 = swz8(r32);
  // X fragment: 16 bytes at k = 64H + 16*hsel and 16 at k = 64H + 32 + 16*hsel
  const int c0 = (4 * H + hsel) ^ sw8;
  const int c1 = (4 * H + 2 + hsel) ^ sw8;
  v8i b[C::FM];
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const uint8_t* row = sb + (wm * C::WTM + i * 32 + r32) * C::XROW;
    v4i lo = *reinterpret_cast<const v4i*>(row + c0 * 16);
    v4i hi = *reinterpret_cast<const v4i*>(row + c1 * 16);
    b[i] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  v8i a[C::FN];
  const uint8_t* wb = sb + C::XBYTES;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const uint8_t* row = wb + (wn * C::WTN + j * 32 + r32) * C::WROW;
    if constexpr (C::WFMT == MXGG_FMT_E2M1) {
      // 32 packed fp4 values: k = 64H + 32*hsel .. +31 -> one 16-byte chunk
      const int c = (2 * H + hsel) ^ swz4(r32);
      v4i lo = *reinterpret_cast<const v4i*>(row + c * 16);
      a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
    } else {
      v4i lo = *reinterpret_cast<const v4i*>(row + c0 * 16);
      v4i hi = *reinterpret_cast<const v4i*>(row + c1 * 16);
      a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
          a[j], b[i], acc[i][j], C::WFMT, MXGG_FMT_E4M3, 2 * H, (int)ws[j], 2 * H, (int)xs[i]);
    }
  }
}

#define MXGG_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")
#define MXGG_BARRIER() asm volatile("s_barrier" ::: "memory")
// All of this wave's LDS reads have returned, then barrier: the stage may be
// overwritten by any wave afterwards.
#define MXGG_RELEASE() asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory")
// Padding that lets in-flight v_mfma_scale instructions read their operands
// before the registers can be rewritten: the compiler does not model the
// scale operands as in-flight reads.
#define MXGG_MFMA_DRAIN() asm volatile("s_nop 15\n\ts_nop 15\n\ts_nop 15\n\ts_nop 15" ::: "memory")

// Reduction over steps [s0, s1) (global 128-element steps) restricted to the
// element range [lo, hi).  Steps that are not fully inside [lo, hi) are masked.
// Two LDS stages.  DW (4-byte aligned scale rows): scales travel through LDS
// with the tiles, so the only vector-memory loads in flight are LDS copies and
// one explicit vmcnt wait per step orders them.  !DW: scales are gathered
// byte-wise into registers one step ahead.
template <class C, bool DW>
__device__ __forceinline__ void mainloop(uint8_t* smem, const Operand& X, const Operand& W,
                                         int s0, int s1, int lo, int hi,
                                         v16f (&acc)[C::FM][C::FN]) {
  if (s0 >= s1) return;
  constexpr int NLOAD = C::QX + C::QW + (DW ? C::QS : 0);
  LoadPlan<C> P;
  make_plan<C>(P, X, W);
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int sh = 8 * (lane >> 5);
  uint32_t xc[C::FM], wc[C::FN], xn[C::FM], wn_[C::FN];
  auto full = [&](int st) { return st * BK >= lo && st * BK + BK <= hi; };

  if (full(s0)) issue_tiles<C, false>(smem, X, W, P, s0, lo, hi);
  else issue_tiles<C, true>(smem, X, W, P, s0, lo, hi);
  if constexpr (DW) issue_scales<C>(smem, X, W, P, s0);
  else load_scales<C, false>(xc, wc, X, W, P, s0);

  for (int st = s0; st < s1; ++st) {
    const int cur = (st - s0) & 1;
    if (st + 1 < s1) {
      uint8_t* nb = smem + (cur ^ 1) * C::STAGE;
      if (full(st + 1)) issue_tiles<C, false>(nb, X, W, P, st + 1, lo, hi);
      else issue_tiles<C, true>(nb, X, W, P, st + 1, lo, hi);
      if constexpr (DW) issue_scales<C>(nb, X, W, P, st + 1);
      else load_scales<C, false>(xn, wn_, X, W, P, st + 1);
      MXGG_WAIT_VM(NLOAD);
    } else {
      MXGG_WAIT_VM(0);
    }
    MXGG_BARRIER();
    const uint8_t* sb = smem + cur * C::STAGE;
    if constexpr (DW) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i)
        xc[i] = *reinterpret_cast<const uint32_t*>(sb + C::XSOFF + (wm * C::WTM + i * 32 + (lane & 31)) * 4);
#pragma unroll
      for (int j = 0; j < C::FN; ++j)
        wc[j] = *reinterpret_cast<const uint32_t*>(sb + C::WSOFF + (wn * C::WTN + j * 32 + (lane & 31)) * 4);
    }
    const bool part = !full(st);
    uint32_t xsh[C::FM], wsh[C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i) {
      uint32_t v = xc[i];
      if (part) v = neutralize(v, st, lo, hi);
      xsh[i] = v >> sh;
    }
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      uint32_t v = wc[j];
      if (part) v = neutralize(v, st, lo, hi);
      wsh[j] = v >> sh;
    }
    mma_half<C, 0>(sb, xsh, wsh, acc);
    mma_half<C, 1>(sb, xsh, wsh, acc);
    MXGG_RELEASE();
    MXGG_MFMA_DRAIN();
    if constexpr (!DW) {
#pragma unroll
      for (int i = 0; i < C::FM; ++i) xc[i] = xn[i];
#pragma unroll
      for (int j = 0; j < C::FN; ++j) wc[j] = wn_[j];
    }
  }
}

// ---------------------------------------------------------------------------
// Software-pipelined main loop (aligned-scale path).
//
// Per 128-element step s (stage s%2 holds step s, step s+1 is in flight):
//   half 0: multiply fragments Fa (k 0..63) while the k 64..127 fragments of
//           the same step are read into Fb;
//   half 1: issue two MFMAs on Fb, then -- while they run -- wait for step
//           s+1 to land, take the workgroup barrier (the one barrier of the
//           step), read step s+1's scales and k 0..63 fragments into Fa,
//           start the global->LDS copies of step s+2 into the stage just
//           released, and issue the remaining MFMAs on Fb.
// Every wave has finished reading stage s%2 (lgkmcnt(0)) before that barrier,
// so after it the stage can be refilled.
// ---------------------------------------------------------------------------

template <class C>
struct Frags {
  v8i a[C::FN];   // W fragments (MFMA A operand)
  v8i b[C::FM];   // X fragments (MFMA B operand)
};

template <class C, int H>
__device__ __forceinline__ void read_frags(const uint8_t* sb, Frags<C>& F) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int hsel = lane >> 5;
  const int r32 = lane & 31;
  const int sw8 = swz8(r32);
  const int c0 = (4 * H + hsel) ^ sw8;
  const int c1 = (4 * H + 2 + hsel) ^ sw8;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const uint8_t* row = sb + (wm * C::WTM + i * 32 + r32) * C::XROW;
    v4i lo = *reinterpret_cast<const v4i*>(row + c0 * 16);
    v4i hi = *reinterpret_cast<const v4i*>(row + c1 * 16);
    F.b[i] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  const uint8_t* wb = sb + C::XBYTES;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const uint8_t* row = wb + (wn * C::WTN + j * 32 + r32) * C::WROW;
    if constexpr (C::WFMT == MXGG_FMT_E2M1) {
      const int c = (2 * H + hsel) ^ swz4(r32);
      v4i lo = *reinterpret_cast<const v4i*>(row + c * 16);
      F.a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
    } else {
      v4i lo = *reinterpret_cast<const v4i*>(row + c0 * 16);
      v4i hi = *reinterpret_cast<const v4i*>(row + c1 * 16);
      F.a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
}

// Scale dwords of the step in stage `sb`, shifted so that op_sel 2*H picks
// the byte of the lane's 32-element block; blocks outside [lo, hi) neutral.
template <class C>
__device__ __forceinline__ void read_scales_raw(const uint8_t* sb, uint32_t (&xs)[C::FM],
                                                uint32_t (&ws)[C::FN]) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
    xs[i] = *reinterpret_cast<const uint32_t*>(sb + C::XSOFF + (wm * C::WTM + i * 32 + (lane & 31)) * 4);
#pragma unroll
  for (int j = 0; j < C::FN; ++j)
    ws[j] = *reinterpret_cast<const uint32_t*>(sb + C::WSOFF + (wn * C::WTN + j * 32 + (lane & 31)) * 4);
}

// Neutralize the blocks of step st outside [lo, hi) and shift so that op_sel
// 2*H picks the byte of the lane's 32-element block.
template <class C>
__device__ __forceinline__ void finish_scales(uint32_t (&xs)[C::FM], uint32_t (&ws)[C::FN], int st,
                                              int lo, int hi) {
  const int sh = 8 * ((threadIdx.x % kWave) >> 5);
  const uint32_t m = outside_mask(st, lo, hi);        // wave-uniform
#pragma unroll
  for (int i = 0; i < C::FM; ++i) xs[i] = ((xs[i] & ~m) | (0x7f7f7f7fu & m)) >> sh;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) ws[j] = ((ws[j] & ~m) | (0x7f7f7f7fu & m)) >> sh;
}

// MFMAs number [B, E) of the half's FM x FN grid (row-major over (i, j)).
template <class C, int H, int B, int E>
__device__ __forceinline__ void mfma_range(const Frags<C>& F, const uint32_t (&xs)[C::FM],
                                           const uint32_t (&ws)[C::FN], v16f (&acc)[C::FM][C::FN]) {
#pragma unroll
  for (int t = B; t < E; ++t) {
    const int i = t / C::FN, j = t % C::FN;
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
        F.a[j], F.b[i], acc[i][j], C::WFMT, MXGG_FMT_E4M3, 2 * H, (int)ws[j], 2 * H, (int)xs[i]);
  }
}

template <class C>
__device__ __forceinline__ void issue_step(uint8_t* sb, const Operand& X, const Operand& W,
                                           const LoadPlan<C>& P, int st, int lo, int hi) {
  issue_tiles_sel<C>(sb, X, W, P, st, lo, hi);
  issue_scales<C>(sb, X, W, P, st);
}

// Keep the MFMA operand registers of a region allocated until the region's
// end.  The compiler does not guard the scale operands of v_mfma_scale_* as
// in-flight reads, so a register freed by an MFMA's last use could otherwise be
// rewritten by the very next VALU instruction while the MFMA still reads it.
template <class FR, int NM, int NN>
__device__ __forceinline__ void hold(const FR& F, const uint32_t (&xs)[NM], const uint32_t (&ws)[NN]) {
#if defined(__HIP_DEVICE_COMPILE__)   // VGPR constraints exist only in the device pass
#pragma unroll
  for (int i = 0; i < NM; ++i) asm volatile("" ::"v"(xs[i]), "v"(F.b[i]));
#pragma unroll
  for (int j = 0; j < NN; ++j) asm volatile("" ::"v"(ws[j]), "v"(F.a[j]));
#endif
}

#define MXGG_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// Scheduling recipe for one region: NM MFMAs with NV VMEM reads and ND DS
// reads spread evenly between them (sched_group_barrier groups, in order).
template <int I, int NM, int NV, int ND>
__device__ __forceinline__ void interleave_step() {
  if constexpr (I < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // 1 MFMA
    constexpr int v = (NV * (I + 1)) / NM - (NV * I) / NM;
    constexpr int d = (ND * (I + 1)) / NM - (ND * I) / NM;
    if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x010, v, 0);   // VMEM (incl. LDS DMA)
    if constexpr (d > 0) __builtin_amdgcn_sched_group_barrier(0x100, d, 0);   // DS reads
    interleave_step<I + 1, NM, NV, ND>();
  }
}

template <int NM, int NV, int ND>
__device__ __forceinline__ void interleave() {
  interleave_step<0, NM, NV, ND>();
}

// One steady-state step st (a next step exists).  Scales of step st are in
// (xs, ws); step st+1's are produced into (xn, wn).  The step ends with a drain
// so that the caller may then overwrite (xs, ws).
template <class C>
__device__ __forceinline__ void pipe_step(uint8_t* smem, const Operand& X, const Operand& W,
                                          const LoadPlan<C>& P, int s0, int st, int lo, int hi,
                                          Frags<C>& Fa, Frags<C>& Fb, uint32_t (&xs)[C::FM],
                                          uint32_t (&ws)[C::FN], uint32_t (&xn)[C::FM],
                                          uint32_t (&wn)[C::FN], v16f (&acc)[C::FM][C::FN]) {
  constexpr int NMMA = C::FM * C::FN;
  constexpr int NEARLY = NMMA >= 8 ? 2 : 1;    // MFMAs of half 1 issued before the barrier
  constexpr int NDS0 = C::FM * 2 + (C::WFMT == MXGG_FMT_E2M1 ? C::FN : C::FN * 2);
  const int cur = (st - s0) & 1;
  uint8_t* sb = smem + cur * C::STAGE;
  uint8_t* nb = smem + (cur ^ 1) * C::STAGE;
  // ---- half 0: MFMAs on Fa, reads of the second half into Fb in between
  read_frags<C, 1>(sb, Fb);
  mfma_range<C, 0, 0, NMMA>(Fa, xs, ws, acc);
  interleave<NMMA, 0, NDS0>();
  MXGG_SCHED_FENCE();
  hold(Fa, xs, ws);
  // ---- half 1
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  mfma_range<C, 1, 0, NEARLY>(Fb, xs, ws, acc);
  MXGG_SCHED_FENCE();
  MXGG_WAIT_VM(0);
  MXGG_BARRIER();
  MXGG_SCHED_FENCE();
  // step st+1's scales and first-half fragments are read before the copies of
  // step st+2 are issued into the stage just released (past the end: zeros,
  // never read).  Reads issued in between those LDS-DMA loads came back
  // corrupted when the compiler gave a read a destination register that a
  // just-issued DMA load used as its offset.
  read_scales_raw<C>(nb, xn, wn);
  read_frags<C, 0>(nb, Fa);
  issue_step<C>(sb, X, W, P, st + 2, lo, hi);
  mfma_range<C, 1, NEARLY, NMMA>(Fb, xs, ws, acc);
  MXGG_SCHED_FENCE();
  hold(Fb, xs, ws);
  MXGG_MFMA_DRAIN();
  MXGG_SCHED_FENCE();
  finish_scales<C>(xn, wn, st + 1, lo, hi);
}

template <class C>
__device__ __forceinline__ void pipe_last(const uint8_t* sb, Frags<C>& Fa, Frags<C>& Fb,
                                          const uint32_t (&xs)[C::FM], const uint32_t (&ws)[C::FN],
                                          v16f (&acc)[C::FM][C::FN]) {
  constexpr int NMMA = C::FM * C::FN;
  read_frags<C, 1>(sb, Fb);
  mfma_range<C, 0, 0, NMMA>(Fa, xs, ws, acc);
  mfma_range<C, 1, 0, NMMA>(Fb, xs, ws, acc);
  MXGG_SCHED_FENCE();
  hold(Fa, xs, ws);
  hold(Fb, xs, ws);
  MXGG_MFMA_DRAIN();
  MXGG_SCHED_FENCE();
}

template <class C>
__device__ __forceinline__ void mainloop_pipe(uint8_t* smem, const Operand& X, const Operand& W,
                                              int s0, int s1, int lo, int hi,
                                              v16f (&acc)[C::FM][C::FN]) {
  if (s0 >= s1) return;
  constexpr int NLOAD = C::QX + C::QW + C::QS;
  LoadPlan<C> P;
  make_plan<C>(P, X, W);

  issue_step<C>(smem, X, W, P, s0, lo, hi);
  if (s0 + 1 < s1) {
    issue_step<C>(smem + C::STAGE, X, W, P, s0 + 1, lo, hi);
    MXGG_WAIT_VM(NLOAD);
  } else {
    MXGG_WAIT_VM(0);
  }
  MXGG_BARRIER();
  Frags<C> Fa, Fb;
  uint32_t xa[C::FM], wa[C::FN], xb[C::FM], wb[C::FN];
  read_scales_raw<C>(smem, xa, wa);
  read_frags<C, 0>(smem, Fa);
  finish_scales<C>(xa, wa, s0, lo, hi);

  // steady state: a next step always exists
  int st = s0;
  for (; st + 1 < s1; ++st) {
    pipe_step<C>(smem, X, W, P, s0, st, lo, hi, Fa, Fb, xa, wa, xb, wb, acc);
    // xb/wb now hold step st+1's scales; move them into the current set only
    // after the step's last MFMAs have read xa/wa (pipe_step ends with a drain)
#pragma unroll
    for (int i = 0; i < C::FM; ++i) xa[i] = xb[i];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) wa[j] = wb[j];
  }
  pipe_last<C>(smem + ((st - s0) & 1) * C::STAGE, Fa, Fb, xa, wa, acc);
  // the zero-filled prefetch past the last step may still be writing LDS:
  // drain it before the workgroup can exit and its LDS be reallocated
  MXGG_WAIT_VM(0);
}

// Store an accumulator tile.  Lane l of fragment (i, j) holds output row
// wm*WTM + 32i + l%32 and columns wn*WTN + 32j + 8(q/4) + 4(l/32) + q%4.
// BF16_ONLY: round to bf16 first whatever the output type (wgrad semantics).
template <class C, bool BF16_ONLY>
__device__ __forceinline__ void store_tile(const v16f (&acc)[C::FM][C::FN], uint8_t* out,
                                           int64_t ldo, int rows, int cols, int out_dtype) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const bool vec = out_dtype == MXGG_DTYPE_F32 ? ((ldo % 4) == 0 && ((uintptr_t)out % 16) == 0)
                                               : ((ldo % 4) == 0 && ((uintptr_t)out % 8) == 0);
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const int r = wm * C::WTM + i * 32 + (lane & 31);
    if (r >= rows) continue;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int c = wn * C::WTN + j * 32 + 8 * q4 + 4 * (lane >> 5);
        float v0 = acc[i][j][4 * q4 + 0], v1 = acc[i][j][4 * q4 + 1];
        float v2 = acc[i][j][4 * q4 + 2], v3 = acc[i][j][4 * q4 + 3];
        if (out_dtype == MXGG_DTYPE_F32) {
          if (BF16_ONLY) {
            v0 = round_bf16(v0); v1 = round_bf16(v1); v2 = round_bf16(v2); v3 = round_bf16(v3);
          }
          float* p = reinterpret_cast<float*>(out) + (int64_t)r * ldo + c;
          if (vec && c + 3 < cols) {
            *reinterpret_cast<float4*>(p) = make_float4(v0, v1, v2, v3);
          } else {
            if (c + 0 < cols) p[0] = v0;
            if (c + 1 < cols) p[1] = v1;
            if (c + 2 < cols) p[2] = v2;
            if (c + 3 < cols) p[3] = v3;
          }
        } else {
          uint32_t w0, w1;
          if (out_dtype == MXGG_DTYPE_BF16) {
            w0 = pack_bf16x2(v0, v1);
            w1 = pack_bf16x2(v2, v3);
          } else {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            h2 a = {(_Float16)v0, (_Float16)v1}, b = {(_Float16)v2, (_Float16)v3};
            w0 = __builtin_bit_cast(uint32_t, a);
            w1 = __builtin_bit_cast(uint32_t, b);
          }
          uint16_t* p = reinterpret_cast<uint16_t*>(out) + (int64_t)r * ldo + c;
          if (vec && c + 3 < cols) {
            *reinterpret_cast<uint2*>(p) = make_uint2(w0, w1);
          } else {
            if (c + 0 < cols) p[0] = (uint16_t)(w0 & 0xffff);
            if (c + 1 < cols) p[1] = (uint16_t)(w0 >> 16);
            if (c + 2 < cols) p[2] = (uint16_t)(w1 & 0xffff);
            if (c + 3 < cols) p[3] = (uint16_t)(w1 >> 16);
          }
        }
      }
    }
  }
}

// Store a 16-bit (bf16 / f16) accumulator tile through LDS so that every
// global store instruction writes whole row segments: each wave transposes its
// WTM x WTN tile into its own LDS area (rows of WTN*2 bytes, 16-byte chunks
// XOR-swizzled by row), then 64 lanes store 64 consecutive 16-byte chunks
// (WTN*2/16 chunks per row).  Tiles larger than the free LDS go in passes of
// whole 32-row fragment rows.  Requires ldo % 8 == 0 and a 16-byte aligned
// `out`; the caller must have drained every LDS-DMA load and the workgroup
// must be past its last main-loop LDS read (this function begins with a
// workgroup barrier).
// Largest divisor of fm not above lim (fragment rows per staging pass).
constexpr int store_pass_rows(int fm, int lim) {
  int best = 1;
  for (int d = 1; d <= fm; ++d)
    if (fm % d == 0 && d <= lim) best = d;
  return best;
}

template <class C>
__device__ __forceinline__ void store_tile_lds(const v16f (&acc)[C::FM][C::FN], uint8_t* smem,
                                               uint8_t* out, int64_t ldo, int rows, int cols,
                                               int out_dtype) {
  constexpr int RB = C::WTN * 2;                 // staged row bytes
  constexpr int NCH = RB / 16;                   // 16-byte chunks per row
  constexpr int AVAIL = 2 * C::STAGE / C::NW;    // LDS bytes per wave
  constexpr int FPP = store_pass_rows(C::FM, AVAIL / (32 * RB));   // fragment rows per pass
  static_assert(FPP >= 1 && C::FM % FPP == 0, "store staging");
  static_assert(64 % NCH == 0, "store row width");
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  uint8_t* area = smem + wave * (FPP * 32 * RB);
#pragma unroll
  for (int i0 = 0; i0 < C::FM; i0 += FPP) {
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < FPP; ++ii) {
      const int m = ii * 32 + (lane & 31);
#pragma unroll
      for (int j = 0; j < C::FN; ++j) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const v16f& a = acc[i0 + ii][j];
          uint32_t w0, w1;
          if (out_dtype == MXGG_DTYPE_BF16) {
            w0 = pack_bf16x2(a[4 * q4 + 0], a[4 * q4 + 1]);
            w1 = pack_bf16x2(a[4 * q4 + 2], a[4 * q4 + 3]);
          } else {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            h2 x = {(_Float16)a[4 * q4 + 0], (_Float16)a[4 * q4 + 1]};
            h2 y = {(_Float16)a[4 * q4 + 2], (_Float16)a[4 * q4 + 3]};
            w0 = __builtin_bit_cast(uint32_t, x);
            w1 = __builtin_bit_cast(uint32_t, y);
          }
          const int c = 4 * j + q4;                      // 16-byte chunk (8 columns)
          *reinterpret_cast<uint2*>(area + m * RB + ((c ^ (m % NCH)) * 16) + 8 * (lane >> 5)) =
              make_uint2(w0, w1);
        }
      }
    }
    __syncthreads();
    constexpr int RPI = 64 / NCH;                        // rows per read instruction
#pragma unroll
    for (int it = 0; it < FPP * 32 / RPI; ++it) {
      const int r = it * RPI + lane / NCH;
      const int c = lane % NCH;
      const uint4 v = *reinterpret_cast<const uint4*>(area + r * RB + ((c ^ (r % NCH)) * 16));
      const int row = wm * C::WTM + i0 * 32 + r;
      const int col = wn * C::WTN + c * 8;
      if (row < rows) {
        uint16_t* p = reinterpret_cast<uint16_t*>(out) + (int64_t)row * ldo + col;
        if (col + 8 <= cols) {
          *reinterpret_cast<uint4*>(p) = v;
        } else {
          const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (col + e < cols) p[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// forward / dgrad
// ---------------------------------------------------------------------------

struct FwdParams {
  const uint8_t* a; int64_t lda; const uint8_t* as; int64_t ldas;
  const uint8_t* b; int64_t ldb_n; int64_t ldb_e; const uint8_t* bs; int64_t ldbs_n; int64_t ldbs_e;
  const int32_t* offs; int E; int64_t M; int64_t N; int64_t K;
  uint8_t* out; int out_dtype; int64_t ldo;
  int grid_n; int group_m; int xcd;
};

template <class C, bool DW>
__global__ __launch_bounds__(C::NT) void fwd_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];
  const int pid = blockIdx.x;
  const int total_m = route_total(p.offs, p.E, C::BM);
  const int tiles = total_m * p.grid_n;
  if (pid >= tiles) return;
  const int t = p.xcd > 1 ? xcd_swizzle(pid, tiles, p.xcd) : pid;
  int pm, pn;
  pid_grid(t, total_m, p.grid_n, p.group_m, pm, pn);
  const TileRoute r = route_find(p.offs, p.E, C::BM, pm);
  if (r.expert < 0) return;
  const int64_t row0 = (int64_t)r.start + (int64_t)r.block * C::BM;
  int64_t rows64 = p.M - row0;
  if (rows64 > r.rows) rows64 = r.rows;
  if (rows64 <= 0) return;
  const int rows = (int)rows64;
  const int64_t n0 = (int64_t)pn * C::BN;
  const int cols = (int)(p.N - n0 < C::BN ? p.N - n0 : C::BN);

  Operand X, W;
  X.ld = (uint32_t)p.lda;
  X.lds = (uint32_t)p.ldas;
  X.data = make_rsrc(p.a + row0 * p.lda, (uint32_t)rows * X.ld);
  X.scale = make_rsrc(p.as + row0 * p.ldas, (uint32_t)rows * X.lds);
  W.ld = (uint32_t)p.ldb_n;
  W.lds = (uint32_t)p.ldbs_n;
  W.data = make_rsrc(p.b + (int64_t)r.expert * p.ldb_e + n0 * p.ldb_n, (uint32_t)cols * W.ld);
  W.scale = make_rsrc(p.bs + (int64_t)r.expert * p.ldbs_e + n0 * p.ldbs_n, (uint32_t)cols * W.lds);

  v16f acc[C::FM][C::FN];
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = (v16f){};

  const int K = (int)p.K;
  if constexpr (DW) mainloop_pipe<C>(smem, X, W, 0, (K + BK - 1) / BK, 0, K, acc);
  else mainloop<C, DW>(smem, X, W, 0, (K + BK - 1) / BK, 0, K, acc);

  const int esz = p.out_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  uint8_t* o = p.out + (row0 * p.ldo + n0) * esz;
  if (DW && esz == 2 && p.ldo % 8 == 0 && (uintptr_t)o % 16 == 0)
    store_tile_lds<C>(acc, smem, o, p.ldo, rows, cols, p.out_dtype);
  else
    store_tile<C, false>(acc, o, p.ldo, rows, cols, p.out_dtype);
}

// ---------------------------------------------------------------------------
// weight gradient: one workgroup per (group, N tile, K tile); the group's
// token range is the reduction range (masked at unaligned ends).
// ---------------------------------------------------------------------------

struct WgradParams {
  const uint8_t* go; int64_t ld_go; const uint8_t* gos; int64_t ld_gos;
  const uint8_t* ia; int64_t ld_ia; const uint8_t* ias; int64_t ld_ias;
  const int32_t* offs; int E; int64_t M; int64_t N; int64_t K;
  uint8_t* out; int out_dtype;
  int tiles_n; int tiles_k;
};

template <class C, bool DW>
__global__ __launch_bounds__(C::NT) void wgrad_kernel(WgradParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * C::STAGE];
  const int g = blockIdx.y;
  const int tn = blockIdx.x / p.tiles_k;       // X side: rows of go_t (output rows n)
  const int tk = blockIdx.x % p.tiles_k;       // W side: rows of ia_t (output cols k)
  int lo = g > 0 ? p.offs[g - 1] : 0;
  int hi = p.offs[g];
  if (lo < 0) lo = 0;
  if (hi > p.M) hi = (int)p.M;
  const int64_t n0 = (int64_t)tn * C::BM, k0 = (int64_t)tk * C::BN;
  const int rows = (int)(p.N - n0 < C::BM ? p.N - n0 : C::BM);
  const int cols = (int)(p.K - k0 < C::BN ? p.K - k0 : C::BN);

  Operand X, W;
  X.ld = (uint32_t)p.ld_go;
  X.lds = (uint32_t)p.ld_gos;
  X.data = make_rsrc(p.go + n0 * p.ld_go, (uint32_t)rows * X.ld);
  X.scale = make_rsrc(p.gos + n0 * p.ld_gos, (uint32_t)rows * X.lds);
  W.ld = (uint32_t)p.ld_ia;
  W.lds = (uint32_t)p.ld_ias;
  W.data = make_rsrc(p.ia + k0 * p.ld_ia, (uint32_t)cols * W.ld);
  W.scale = make_rsrc(p.ias + k0 * p.ld_ias, (uint32_t)cols * W.lds);

  v16f acc[C::FM][C::FN];
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = (v16f){};

  if (hi > lo) {
    if constexpr (DW) mainloop_pipe<C>(smem, X, W, lo / BK, (hi + BK - 1) / BK, lo, hi, acc);
    else mainloop<C, DW>(smem, X, W, lo / BK, (hi + BK - 1) / BK, lo, hi, acc);
  }

  const int esz = p.out_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  uint8_t* o = p.out + ((int64_t)g * p.N * p.K + n0 * p.K + k0) * esz;
  if (DW && esz == 2 && p.K % 8 == 0 && (uintptr_t)o % 16 == 0)
    store_tile_lds<C>(acc, smem, o, p.K, rows, cols, p.out_dtype);
  else
    store_tile<C, true>(acc, o, p.K, rows, cols, p.out_dtype);
}

// ---------------------------------------------------------------------------
// routing table / schedule (test hooks exposing the in-kernel device code)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(64) void routing_kernel(const int32_t* offs, int E, int BM,
                                                     int grid_m_ub, int32_t* out) {
  // one wave; hist / start rows then the pid map
  for (int e = threadIdx.x; e < E; e += kWave) {
    int prev = e > 0 ? offs[e - 1] : 0;
    out[e] = offs[e] - prev;
    out[E + e] = prev;
  }
  const int total = route_total(offs, E, BM);
  if (threadIdx.x == 0) out[2 * E] = total;
  for (int base = 0; base < grid_m_ub; base += kWave) {
    // every lane resolves a different pid; route_find is wave-collective, so
    // loop over the wave's pids one at a time
    for (int k = 0; k < kWave && base + k < grid_m_ub; ++k) {
      int pid = base + k;
      int v = -1;
      if (pid < total) {
        TileRoute r = route_find(offs, E, BM, pid);
        if (r.expert >= 0) v = (r.block << 16) | r.expert;
      }
      if (threadIdx.x == 0) out[2 * E + 1 + pid] = v;
    }
  }
}

__global__ __launch_bounds__(64) void schedule_kernel(const int32_t* offs, int E, int BM,
                                                      int grid_n, int group_m, int xcd,
                                                      int programs, int32_t* out) {
  const int total_m = route_total(offs, E, BM);
  const int tiles = total_m * grid_n;
  for (int pid = threadIdx.x; pid < programs; pid += kWave) {
    int pm = -1, pn = -1;
    if (pid < tiles) {
      int t = xcd > 1 ? xcd_swizzle(pid, tiles, xcd) : pid;
      pid_grid(t, total_m, grid_n, group_m, pm, pn);
    }
    out[2 * pid] = pm;
    out[2 * pid + 1] = pn;
  }
}

}  // namespace mxgg

// ===========================================================================
// C ABI
// ===========================================================================

using namespace mxgg;

namespace {

typedef Cfg<256, 256, 2, 2, MXGG_FMT_E4M3> CfgF8_256;
typedef Cfg<128, 128, 2, 2, MXGG_FMT_E4M3> CfgF8_128;
typedef Cfg<256, 256, 2, 2, MXGG_FMT_E2M1> CfgF4_256;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct FwdChoice {
  int bm, bn, group_m, xcd;
};

FwdChoice pick_fwd(int E, int64_t M, int64_t N, int64_t K, int b_fmt, int bm, int bn, int gm,
                   int xcd) {
  (void)E; (void)M; (void)K;
  FwdChoice c{256, 256, 8, 8};
  if (b_fmt == MXGG_FMT_E4M3 && N <= 2048 && K <= 2048) { c.bm = 128; c.bn = 128; }
  if (bm) c.bm = bm;
  if (bn) c.bn = bn;
  if (gm) c.group_m = gm;
  if (xcd) c.xcd = xcd;
  return c;
}

template <class C>
int launch_fwd(const FwdParams& p0, int grid_m_ub, int gm, int xcd, bool dw, hipStream_t st) {
  FwdParams p = p0;
  p.grid_n = (int)cdiv(p.N, C::BN);
  p.group_m = gm;
  p.xcd = xcd;
  const int64_t grid = (int64_t)grid_m_ub * p.grid_n;
  if (grid <= 0) return MXGG_OK;
  if (grid > INT32_MAX) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: grid too large");
  if (dw) hipLaunchKernelGGL((fwd_kernel<C, true>), dim3((unsigned)grid), dim3(C::NT), 0, st, p);
  else hipLaunchKernelGGL((fwd_kernel<C, false>), dim3((unsigned)grid), dim3(C::NT), 0, st, p);
  return launch_status("grouped_mm");
}

}  // namespace

extern "C" int64_t mxgg_routing_words(int E, int64_t M, int block_m) {
  if (E <= 0 || M < 0 || block_m <= 0) return 0;
  return 2 * (int64_t)E + 1 + cdiv(M, block_m) + (E > 1 ? E - 1 : 0);
}

extern "C" int mxgg_build_routing(const int32_t* offs, int E, int64_t M, int block_m, int32_t* out,
                                  void* stream) {
  clear_error();
  if (E <= 0 || E > 65535) return fail(MXGG_ERR_INVALID_ARG, "build_routing: E=%d out of range", E);
  if (M < 0 || M > INT32_MAX) return fail(MXGG_ERR_INVALID_ARG, "build_routing: M out of range");
  if (block_m <= 0) return fail(MXGG_ERR_INVALID_ARG, "build_routing: block_m must be positive");
  if (!offs || !out) return fail(MXGG_ERR_INVALID_ARG, "build_routing: null pointer");
  if (int rc = require_device()) return rc;
  const int64_t ub = cdiv(M, block_m) + (E > 1 ? E - 1 : 0);
  hipLaunchKernelGGL(routing_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, offs, E, block_m,
                     (int)ub, out);
  return launch_status("build_routing");
}

extern "C" int64_t mxgg_schedule_programs(int E, int64_t M, int64_t N, int block_m, int block_n) {
  if (E <= 0 || M < 0 || N < 0 || block_m <= 0 || block_n <= 0) return 0;
  return (cdiv(M, block_m) + (E > 1 ? E - 1 : 0)) * cdiv(N, block_n);
}

extern "C" int mxgg_tile_schedule(const int32_t* offs, int E, int64_t M, int64_t N, int block_m,
                                  int block_n, int group_m, int xcd_swizzle, int32_t* out,
                                  void* stream) {
  clear_error();
  if (E <= 0 || E > 65535) return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: E=%d out of range", E);
  if (block_m <= 0 || block_n <= 0 || group_m <= 0 || xcd_swizzle <= 0)
    return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: block sizes, group_m and xcd_swizzle must be positive");
  const int64_t programs = mxgg_schedule_programs(E, M, N, block_m, block_n);
  if (programs > INT32_MAX) return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: too many programs");
  if (!offs || !out) return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: null pointer");
  if (int rc = require_device()) return rc;
  hipLaunchKernelGGL(schedule_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, offs, E, block_m,
                     (int)cdiv(N, block_n), group_m, xcd_swizzle, (int)programs, out);
  return launch_status("tile_schedule");
}

static bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

extern "C" int mxgg_grouped_mm(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas,
                               const uint8_t* B, int b_fmt, int64_t ldb_n, int64_t ldb_e,
                               const uint8_t* B_s, int64_t ldbs_n, int64_t ldbs_e,
                               const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                               void* out, int out_dtype, int64_t ldo, int block_m, int block_n,
                               int group_m, int xcd, void* stream) {
  clear_error();
  if (b_fmt != MXGG_FMT_E4M3 && b_fmt != MXGG_FMT_E2M1)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: weight format %d not E4M3/E2M1", b_fmt);
  if (out_dtype != MXGG_DTYPE_BF16 && out_dtype != MXGG_DTYPE_F16 && out_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: out_dtype %d not BF16/F16/F32", out_dtype);
  if (E <= 0 || E > 65535) return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: E=%d out of range", E);
  if (M < 0 || N < 0 || K < 0) return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: negative shape");
  if (K % 32) return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: K=%lld must be a multiple of 32", (long long)K);
  if (b_fmt == MXGG_FMT_E2M1 && K % 128)
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: e2m1 weights need K %% 128 == 0");
  const int64_t kb = b_fmt == MXGG_FMT_E2M1 ? K / 2 : K;
  if (lda < K || ldas < K / 32 || ldb_n < kb || ldbs_n < K / 32 || ldo < N)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: a row stride is smaller than its row");
  if (E > 1 && (ldb_e < N * ldb_n || ldbs_e < N * ldbs_n))
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: expert stride smaller than one expert");
  if (lda % 16 || ldb_n % 16 || !aligned16(A) || !aligned16(B))
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: A/B rows must be 16-byte aligned");
  if (lda >= (1 << 23) || ldb_n >= (1 << 23) || ldas >= (1 << 23) || ldbs_n >= (1 << 23))
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: row strides must be below 2**23 bytes");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: dimension above 2**31");
  if (M == 0 || N == 0) return MXGG_OK;
  if (!A || !A_s || !B || !B_s || !offs || !out)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: null pointer");
  if (int rc = require_device()) return rc;
  FwdChoice c = pick_fwd(E, M, N, K, b_fmt, block_m, block_n, group_m, xcd);
  const bool dw = (ldas % 4 == 0) && (ldbs_n % 4 == 0) && (ldbs_e % 4 == 0) &&
                  ((uintptr_t)A_s % 4 == 0) && ((uintptr_t)B_s % 4 == 0);
  FwdParams p{A, lda, A_s, ldas, B, ldb_n, ldb_e, B_s, ldbs_n, ldbs_e, offs, E, M, N, K,
              (uint8_t*)out, out_dtype, ldo, 0, 0, 0};
  hipStream_t st = (hipStream_t)stream;
  if (b_fmt == MXGG_FMT_E2M1) {
    if (c.bm != 256 || c.bn != 256) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: e2m1 build has 256x256 tiles only");
    return launch_fwd<CfgF4_256>(p, (int)(cdiv(M, 256) + E - 1), c.group_m, c.xcd, dw, st);
  }
  if (c.bm == 256 && c.bn == 256)
    return launch_fwd<CfgF8_256>(p, (int)(cdiv(M, 256) + E - 1), c.group_m, c.xcd, dw, st);
  if (c.bm == 128 && c.bn == 128)
    return launch_fwd<CfgF8_128>(p, (int)(cdiv(M, 128) + E - 1), c.group_m, c.xcd, dw, st);
  return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: tile %dx%d not built (256x256, 128x128)", c.bm, c.bn);
}

extern "C" int mxgg_grouped_mm_config(int E, int64_t M, int64_t N, int64_t K, int b_fmt, int* block_m,
                                      int* block_n, int* group_m, int* xcd_swizzle) {
  clear_error();
  if (!block_m || !block_n || !group_m || !xcd_swizzle)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm_config: null output pointer");
  if (b_fmt != MXGG_FMT_E4M3 && b_fmt != MXGG_FMT_E2M1)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm_config: weight format %d not E4M3/E2M1", b_fmt);
  FwdChoice c = pick_fwd(E, M, N, K, b_fmt, *block_m, *block_n, *group_m, *xcd_swizzle);
  *block_m = c.bm;
  *block_n = c.bn;
  *group_m = c.group_m;
  *xcd_swizzle = c.xcd;
  const bool built = b_fmt == MXGG_FMT_E2M1 ? (c.bm == 256 && c.bn == 256)
                                           : ((c.bm == 256 && c.bn == 256) || (c.bm == 128 && c.bn == 128));
  if (!built) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm_config: tile %dx%d not built", c.bm, c.bn);
  return MXGG_OK;
}

extern "C" size_t mxgg_wgrad_workspace_size(int E, int64_t M, int64_t N, int64_t K) {
  (void)E; (void)M; (void)N; (void)K;
  return 0;
}

extern "C" int mxgg_wgrad(const uint8_t* go_t, int64_t ld_go, const uint8_t* go_s, int64_t ld_gos,
                          const uint8_t* ia_t, int64_t ld_ia, const uint8_t* ia_s, int64_t ld_ias,
                          const int32_t* offs, int E, int64_t M, int64_t N, int64_t K, void* out,
                          int out_dtype, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  (void)workspace; (void)ws_bytes;
  if (out_dtype != MXGG_DTYPE_BF16 && out_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: out_dtype %d not BF16/F32", out_dtype);
  if (E <= 0 || E > 65535) return fail(MXGG_ERR_INVALID_ARG, "wgrad: E=%d out of range", E);
  if (M < 0 || N < 0 || K < 0) return fail(MXGG_ERR_INVALID_ARG, "wgrad: negative shape");
  if (M % 32) return fail(MXGG_ERR_INVALID_ARG, "wgrad: M=%lld must be a multiple of 32", (long long)M);
  if (ld_go < M || ld_ia < M || ld_gos < M / 32 || ld_ias < M / 32)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: a row stride is smaller than its row");
  if (ld_go % 16 || ld_ia % 16 || !aligned16(go_t) || !aligned16(ia_t))
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: operand rows must be 16-byte aligned");
  if (ld_go >= (1 << 23) || ld_ia >= (1 << 23) || ld_gos >= (1 << 23) || ld_ias >= (1 << 23))
    return fail(MXGG_ERR_UNSUPPORTED, "wgrad: row strides must be below 2**23 bytes");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXGG_ERR_UNSUPPORTED, "wgrad: dimension above 2**31");
  if (N == 0 || K == 0) return MXGG_OK;
  if (!go_t || !go_s || !ia_t || !ia_s || !offs || !out)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: null pointer");
  if (int rc = require_device()) return rc;
  typedef CfgF8_256 C;
  WgradParams p{go_t, ld_go, go_s, ld_gos, ia_t, ld_ia, ia_s, ld_ias, offs, E, M, N, K,
                (uint8_t*)out, out_dtype, (int)cdiv(N, C::BM), (int)cdiv(K, C::BN)};
  const bool dw = (ld_gos % 4 == 0) && (ld_ias % 4 == 0) && ((uintptr_t)go_s % 4 == 0) &&
                  ((uintptr_t)ia_s % 4 == 0);
  const int64_t gx = (int64_t)p.tiles_n * p.tiles_k;
  if (gx > INT32_MAX) return fail(MXGG_ERR_UNSUPPORTED, "wgrad: grid too large");
  dim3 grid((unsigned)gx, (unsigned)E);
  hipStream_t st = (hipStream_t)stream;
  if (dw) hipLaunchKernelGGL((wgrad_kernel<C, true>), grid, dim3(C::NT), 0, st, p);
  else hipLaunchKernelGGL((wgrad_kernel<C, false>), grid, dim3(C::NT), 0, st, p);
  return launch_status("wgrad");
}
