// MX-scaled grouped GEMM kernels for gfx950 (CDNA4):
//   * forward / dgrad:  out[s:e] = A[s:e] @ B[g]^T          (kernels/forward.py:81-294)
//   * weight gradient:  out[g]   = GO[:, s:e] @ IA[:, s:e]^T (kernels/backward.py:31-215)
//   * routing table and tile schedule exposed for testing   (kernels/forward.py:31-51, 296-365)
//   * scale re-layout feeding both GEMMs                    (the role of kernels/forward.py:367-397)
//   * split of an under-filled last round along the reduction, with fp32
//     partial tiles and a reduce kernel        (generalises kernels/backward.py:106-215)
//   * forward last round with a reduction too short to split as 128 x 128
//     quarter tiles (fwd_quad_kernel)
//
// Both GEMMs are "NT" products whose two operands are contiguous along the
// reduction dimension, so they share one main loop:
//   acc[r][c] = sum_k X[r][k] * W[c][k] * 2**(xs[r][k/32]-127) * 2**(ws[c][k/32]-127)
// with X on the B side and W on the A side of v_mfma_scale_f32_32x32x64_f8f6f4,
// so that every lane of the accumulator holds 4 consecutive output columns.
//
// Main loop (ring_mainloop): the reduction runs in 64-element stages held in
// an NS-deep LDS ring.  While stage s is multiplied out of registers, stage
// s+1 is read from LDS and stages s+2 .. s+NS are in flight, so the copies of
// a stage have NS-1 stage times to land and the copy engine always has
// several stages queued.  (The two 64-byte halves of a 128-byte line, copied
// a stage apart, move at ~80% of the full-line rate; copying stages in pairs
// recovers the rate but shortens the prefetch, and measured slower.)
//   * X and W tiles go global -> LDS directly with 16-byte buffer_load ... lds;
//     chunks outside the reduction range read as zero through the buffer
//     range check.  LDS rows are 64 bytes (e4m3) or 32 bytes (packed e2m1)
//     with 16-byte chunks XOR-swizzled by row: conflict-free fragment reads.
//   * e8m0 scales: a re-layout kernel first writes the plain `to_mx` scales
//     step-major, one dword (4 scale bytes = one 128-element step) per row:
//     [step][row].  The scales of a tile for two steps are then a few
//     contiguous 1 KB pieces, copied into a two-slot scale ring every four
//     stages; each MFMA takes its lane's byte at op_sel 0.
//   * one workgroup barrier per stage; fragment and scale registers alternate
//     between two sets (loop body unrolled twice).
#include <mutex>
#include <type_traits>

#include "mxgg_device.h"
#include "mxgg_host.h"

namespace mxgg {

constexpr int BKS = 64;        // reduction elements per stage
constexpr int STEP = 128;      // reduction elements per scale dword (4 blocks of 32)
constexpr int SCG = 2;         // steps per step-major scale group (one scale-ring slot)

// Split of the last, partial round.  With T tiles and P workgroups resident
// at once, the rem = T % P tiles of the last round leave most of the chip idle
// for (a fraction of) a tile time.  They can instead be cut into S pieces
// along the reduction (whole 128-element steps, at least kMinSplitSteps per
// piece, at most kMaxSplit pieces per tile, `slots` pieces in all); pieces
// store fp32 partial tiles and a second kernel adds them in piece order and
// rounds once.  Tiles 0 .. dp-1 run whole, tile dp + v as pieces v*S ..
// v*S+S-1.  Up to P / 2 last-round tiles, S <= P / rem keeps the pieces in one
// round.  Past that, S pieces per tile run in ceil(rem * S / P) rounds (160
// tiles on 256 CUs: 3 pieces each, two rounds of a third of the reduction
// instead of one round of all of it).
//
// Only a last round that follows at most kSplitMaxRounds full rounds is
// split (measured: a loss from 5 full rounds on).  Tiles of one launch stay
// in step round after round, so the last round does leave most CUs idle,
// but its few tiles run uncontended at a higher clock, in about 0.6 of a
// full round's tile time, and the pieces, the reduce and two more launches
// cost as much.  S is picked by a cost model
// (nanoseconds, MI355X kernel traces): the last round of n steps costs about
// kTailNsPerStep * n (0.75 of 1.7 us per step; kBusyNsPerStep, 1.7 us, when
// the last round fills more than half the chip); cut into S pieces it costs
// rounds * n / S of that, plus kSplitFixedNs (piece prologue and epilogue, two
// launches) plus the partial traffic, rem * S tiles written and read back
// (kSplitNsPerMiB).  No split unless that saves at least kSplitMinGainNs (the
// model is coarse); reductions shorter than kMinSplitTotal steps are never
// split.  Integer arithmetic: every kernel that recomputes the plan on the
// device gets the same answer, bit for bit.
constexpr int kMinSplitSteps = 4;
constexpr int kMaxSplit = 8;
constexpr int kMinSplitTotal = 32;
constexpr int kSplitMaxRounds = 2;
constexpr int64_t kTailNsPerStep = 1275;
constexpr int64_t kBusyNsPerStep = 1700;
constexpr int64_t kSplitFixedNs = 9000;
constexpr int64_t kSplitNsPerMiB = 400;
constexpr int64_t kSplitMinGainNs = 16000;
constexpr size_t kSplitBytes = (size_t)128 << 20;  // partial-tile area of a full workspace

struct Split {
  int dp;       // tiles computed whole
  int S;        // pieces per split tile (1: no split)
  int units;    // pieces in all (rem * S, or 0)
};

__host__ __device__ inline Split split_plan(int T, int P, int nsteps, int slots, int tile_kib) {
  Split sp{T, 1, 0};
  if (T <= 0 || P <= 0 || nsteps < kMinSplitTotal || T / P > kSplitMaxRounds) return sp;
  const int rem = T % P;
  if (rem == 0) return sp;
  int smax = 2 * rem > P ? kMaxSplit : P / rem;
  if (smax > kMaxSplit) smax = kMaxSplit;
  if (smax > nsteps / kMinSplitSteps) smax = nsteps / kMinSplitSteps;
  if (smax > slots / rem) smax = slots / rem;
  // int32 throughout: tail <= 1700 * 2^20, rounds * (tail / S) <= tail, and
  // rem * S <= slots <= 4096 with tile_kib <= 256 keeps the staging term
  // below 2^30.  Unrolled, every
  // tail / S has a constant divisor.
  const int per = (int)(2 * rem > P ? kBusyNsPerStep : kTailNsPerStep);
  const int tail = per * (nsteps < (1 << 20) ? nsteps : (1 << 20));
  int best = (int)kSplitMinGainNs;
#pragma unroll
  for (int S = 2; S <= kMaxSplit; ++S) {
    if (S > smax) break;
    const int rounds = (rem * S + P - 1) / P;   // <= S while rem < P
    const int gain =
        tail - rounds * (tail / S) - (int)kSplitFixedNs - rem * S * tile_kib * (int)kSplitNsPerMiB / 1024;
    if (gain > best) {
      best = gain;
      sp.S = S;
    }
  }
  if (sp.S < 2) return sp;
  sp.dp = T - rem;
  sp.units = rem * sp.S;
  return sp;
}

// Steps [a, b) of piece s out of S over steps [a0, a0 + n).  32-bit
// unsigned arithmetic: n < 2**25 steps and s < S <= kMaxSplit keep n * (s+1)
// below 2**28 (a 64-bit division is a long software sequence on the device).
__host__ __device__ inline void split_range(int a0, int n, int s, int S, int& a, int& b) {
  a = a0 + (int)((uint32_t)n * (uint32_t)s / (uint32_t)S);
  b = a0 + (int)((uint32_t)n * (uint32_t)(s + 1) / (uint32_t)S);
}

template <int BM_, int BN_, int WGM_, int WGN_, int WFMT_, int NS_, bool PS_ = false>
struct Cfg {
  static constexpr int BM = BM_;        // X rows per tile (output rows)
  static constexpr int BN = BN_;        // W rows per tile (output columns)
  static constexpr int WGM = WGM_;      // waves along rows
  static constexpr int WGN = WGN_;      // waves along columns
  static constexpr int WFMT = WFMT_;    // W element format (X is always e4m3)
  static constexpr int NS = NS_;        // ring depth (stages)
  // Scale source: false, step-major dwords [step][row] (the re-layout
  // kernel's output or the quantizer's native layout); true, the plain
  // to_mx scales (row r's byte b at r * ld + b, ld a multiple of 16), read
  // directly in 32-byte row pieces of 8 steps.
  static constexpr bool PS = PS_;
  static constexpr bool XD = false;     // X in two-stage slots (XLine)
  static constexpr bool F4 = WFMT == MXGG_FMT_E2M1;
  static constexpr int NW = WGM * WGN;
  static constexpr int NT = NW * kWave;
  static constexpr int WTM = BM / WGM;
  static constexpr int WTN = BN / WGN;
  static constexpr int FM = WTM / 32;
  static constexpr int FN = WTN / 32;
  static constexpr int XROW = BKS;                  // bytes per X row per stage
  static constexpr int WROW = F4 ? BKS / 2 : BKS;   // bytes per W row per stage
  static constexpr int XBYTES = BM * XROW;
  static constexpr int WBYTES = BN * WROW;
  static constexpr int STAGE = XBYTES + WBYTES;
  // scale ring after the data ring: two slots of GSTEPS steps each.
  // Step-major: GSTEPS x BM X-row dwords ([step][row]) followed by GSTEPS x
  // BN W-row dwords.  Plain: BM X rows then BN W rows of 32 bytes (steps
  // 8c .. 8c+7 of the row, c = the group's chunk of the reduction), the two
  // 16-byte halves of rows 8..15 of every 16 swapped (conflict-free reads of
  // one step over 32 rows, two ways apart at most).
  static constexpr int GSTEPS = PS ? 8 : SCG;           // steps per scale group (slot)
  static constexpr int GSTAGES = GSTEPS * STEP / BKS;   // stages per scale group
  static constexpr int SSLOT = GSTEPS * (BM + BN) * 4;
  static constexpr int SOFF = NS * STAGE;
  static constexpr int LDS = SOFF + 2 * SSLOT;
  static constexpr int QX = XBYTES / 1024 / NW;     // 1 KB data copies per wave and stage
  static constexpr int QW = WBYTES / 1024 / NW;
  static constexpr int LPS = QX + QW;               // LDS-DMA loads per wave and stage
  // step-major: 1 KB scale copies of the X part (waves 0 ..) and per group
  static constexpr int NSX = PS ? 0 : SCG * BM * 4 / 1024;
  static constexpr int NSD = PS ? 0 : SSLOT / 1024;
  // plain: 1 KB scale copies (32 rows) per wave and group; waves 0 .. NXW-1
  // copy X rows, the others W rows
  static constexpr int SPW = PS ? (BM + BN) / 32 / NW : 0;
  static constexpr int NXW = PS ? BM / 32 / SPW : 0;
  static_assert(XBYTES % (1024 * NW) == 0 && WBYTES % (1024 * NW) == 0, "tile/wave split");
  static_assert(PS || ((SCG * BM * 4) % 1024 == 0 && (SCG * BN * 4) % 1024 == 0 && NSD <= NW),
                "scale copies: one operand each, at most one per wave");
  static_assert(!PS || (SPW >= 1 && (BM + BN) % (32 * NW) == 0 && (BM / 32) % SPW == 0),
                "plain scale copies: whole 32-row pieces, one operand per wave");
  static_assert(BM % 4 == 0 && BN % 4 == 0, "scale pieces stay in one step");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  static_assert(NS >= 3 && LDS <= 160 * 1024, "ring depth / LDS budget");
  // a scale group is copied GSTAGES - 1 stages (or more) before its first
  // read; the wait before that read covers it only if the stage read then was
  // issued no earlier than the group
  static_assert(NS <= GSTAGES + 1, "ring deeper than the scale prefetch");
  static_assert((NS - 1) * LPS + 2 * (PS ? SPW : 1) <= 63, "vmcnt range");
};

// Configuration B with X in two-stage slots.  A row-major X row gives a
// stage 64 bytes, half a 128-byte line, so the one-stage ring copies each X
// line in two requests.  X slot q here holds stages 2q and 2q+1 of every
// tile row as one 128-byte piece, copied as whole lines; W keeps one-stage
// slots.  B::NS slots of each, in two regions (256 x 256 tiles: X 96 KB,
// W 48 KB), then the step-major scale ring.  Slot layout: tile row m at
// byte 128 m, its 16-byte unit u (stage 2q + u / 4, elements 16 (u % 4) ..
// +15 of it) at unit u ^ (m % 8) ^ ((m / 8) % 2): one unit over 8 consecutive
// rows hits 8 different 16-byte bank groups of 128 bytes, and over 16
// consecutive rows 16 different ones of 256 bytes.
template <class B>
struct XLine : B {
  static constexpr bool XD = true;
  static constexpr int XSLOT = 2 * B::XBYTES;
  static constexpr int WOFF = B::NS * XSLOT;
  static constexpr int SOFF = WOFF + B::NS * B::WBYTES;
  static constexpr int LDS = SOFF + 2 * B::SSLOT;
  static_assert(!B::PS && !B::F4 && B::NS == 3, "two-stage X slots: e4m3, step-major scales, 3 slots");
  static_assert(B::QX % 2 == 0, "even and odd X copies alternate in a half pair");
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(3 * B::QX + 2 * B::QW + 2 <= 63, "vmcnt range");
};

// 16-byte chunk swizzles: bijective on the chunk index for every 8-row and
// every 16-row class, 64-byte rows (swz4) and 32-byte rows (swz2).  Both
// depend on row % 16 only.
__device__ __forceinline__ int swz4(int r) {
  return ((((r >> 2) ^ (r >> 3)) & 1) << 1) | (((r >> 1) ^ (r >> 2)) & 1);
}
__device__ __forceinline__ int swz2(int r) { return ((r >> 2) ^ (r >> 3)) & 1; }

// A tile's rows of one operand in global memory, in one of three layouts,
// G = 2**pl rows per group:
//   rows  (pl = 0): byte k of row r at r * ld + k;
//   pairs (pl = 1, e4m3) and quads (pl = 2, packed e2m1): the G rows of a
//         group interleave in P = 128 / G byte pieces -- one 64-element
//         stage of a row -- byte k of row r at (r / G) * G ld +
//         (k / P) * 128 + (r % G) * P + k % P, so the stage pieces of a group
//         fill one 128-byte line and a copy touches whole lines instead of
//         halves (pairs) or quarters (quads).
// Local row r of the tile is row e = r + shift of the buffer `data`, which
// starts at the group of the tile's first row (shift = row0 % G); the range
// ends after the group of the tile's last row, so reads past the tile's rows
// return 0 except the other rows of that last group.
struct Operand {
  __amdgpu_buffer_rsrc_t data;
  uint32_t ld;                   // bytes between rows (groups: between groups / G)
  uint32_t pl;                   // log2 G: 0 rows, 1 pairs, 2 quads
  uint32_t shift;                // row0 % G of the tile
};

// Operand of rows row0 .. row0 + rows - 1 of the matrix at `base`.
__device__ __forceinline__ Operand make_operand(const uint8_t* base, int64_t ld, int pl, int64_t row0, int rows) {
  Operand o;
  o.ld = (uint32_t)ld;
  o.pl = (uint32_t)pl;
  const int64_t mask = ((int64_t)1 << pl) - 1;
  o.shift = (uint32_t)(row0 & mask);
  const int64_t unit = ld << pl;                                  // bytes per group
  const uint32_t units = (uint32_t)(((int64_t)o.shift + rows + mask) >> pl);
  o.data = make_rsrc(base + (row0 >> pl) * unit, units * (uint32_t)unit);
  return o;
}

// Byte offset in O.data of byte `col` of local row `row` (pieces of
// 2**pb = 128 / G bytes; for rows, pb = 7 leaves col unchanged).
__device__ __forceinline__ uint32_t operand_off(const Operand& O, uint32_t row, uint32_t col) {
  const uint32_t e = row + O.shift;
  const uint32_t pb = 7u - O.pl;
  return (e >> O.pl) * (O.ld << O.pl) + ((col >> pb) << 7) + ((e & ((1u << O.pl) - 1u)) << pb) +
         (col & ((1u << pb) - 1u));
}

// Where a tile's step-major scales live: dword (t, r) of an operand with R
// rows per step is at byte 4 (t R + r) of the buffer `rsrc` (the operand's
// [step][row] array, re-laid into the workspace or written so by the
// quantizer); reads past the buffer return 0.
struct ScaleSrc {
  __amdgpu_buffer_rsrc_t rsrc;
  uint32_t rows;    // step-major: R, rows per step of that array; plain: bytes per row
  uint32_t row0;    // first row of the tile
};

template <class C>
struct Frags {
  v8i a[C::FN];   // W fragments (MFMA A operand)
  v8i b[C::FM];   // X fragments (MFMA B operand)
};

// Per-lane copy plan.  Data copy i of a wave covers rows q*R .. q*R+R-1
// (q = wave*Q + i; R = 16 rows of 64 bytes, or 32 rows of 32 bytes for packed
// e2m1 W); the lane's row inside a copy and its swizzled chunk do not depend
// on i, so one per-lane offset serves all copies and the row step of copy i
// (R rows: R * ld bytes in either layout, R being even) travels in the scalar
// offset.  The chunk index rides in bits 28..31 (a lane's offset is at most
// 31 rows, or 8 pairs, of a stride below 2**23 plus 112 bytes: below 2**28).
// Scale copy of wave w, step-major (w < NSD): slot dwords 256 w .. 256 w +
// 255, 4 per lane, of the X part (w < NSX) or the W part; lane l covers step
// u and tile rows r .. r+3 of its operand, at byte s_base + t * s_step of that
// operand's scale buffer for step t of the reduction.  Plain: copy i of wave
// w fills slot rows 32 (w SPW + i) .. +31 (X rows for w < NXW, then W rows);
// lane l holds 16 bytes of row l / 2 of the copy, the half (l ^ (l >> 4)) & 1
// of the row's 32-byte piece, at byte s_base + i * s_step + 4 t of that
// operand's scales for the piece starting at step t.
// Two-stage X slots (C::XD): copy c of a pair covers tile rows 8c .. 8c+7
// (128 bytes each), lane l row l / 8 of the copy and slot unit l % 8, which
// holds unit (l % 8) ^ (l / 8) of the row's piece for even c (xoff) and
// that ^ 1 for odd c (xoff2).
template <class C>
struct Plan {
  uint32_t xoff;
  uint32_t xoff2;
  uint32_t woff;
  uint32_t s_base;
  uint32_t s_step;
};

template <class C>
__device__ __forceinline__ void make_plan(Plan<C>& P, const Operand& X, const Operand& W,
                                          const ScaleSrc& xs, const ScaleSrc& ws) {
  const int lane = threadIdx.x % kWave;
  if constexpr (C::XD) {
    const int row = lane / 8;
    const int ue = (lane & 7) ^ row, uo = ue ^ 1;
    P.xoff = operand_off(X, (uint32_t)row, (uint32_t)ue * 16u) | ((uint32_t)ue << 28);
    P.xoff2 = operand_off(X, (uint32_t)row, (uint32_t)uo * 16u) | ((uint32_t)uo << 28);
  } else {
    const int row = lane / 4;
    const int c = (lane & 3) ^ swz4(row);
    P.xoff = operand_off(X, (uint32_t)row, (uint32_t)c * 16u) | ((uint32_t)c << 28);
    P.xoff2 = 0;
  }
  if constexpr (C::F4) {
    const int row = lane / 2;
    const int c = (lane & 1) ^ swz2(row);
    P.woff = operand_off(W, (uint32_t)row, (uint32_t)c * 16u) | ((uint32_t)c << 28);
  } else {
    const int row = lane / 4;
    const int c = (lane & 3) ^ swz4(row);
    P.woff = operand_off(W, (uint32_t)row, (uint32_t)c * 16u) | ((uint32_t)c << 28);
  }
  const int wave = wave_id();
  if constexpr (C::PS) {
    const bool isx = wave < C::NXW;
    const ScaleSrc& S = isx ? xs : ws;
    const int row = (isx ? wave : wave - C::NXW) * C::SPW * 32 + lane / 2;   // operand row of the tile
    const int h = (lane ^ (lane >> 4)) & 1;
    P.s_step = S.rows * 32u;
    P.s_base = (S.row0 + (uint32_t)row) * S.rows + (uint32_t)h * 16u;
  } else {
    const bool isx = wave < C::NSX;
    const int R = isx ? C::BM : C::BN;              // tile rows of the lane's operand
    const int q = (isx ? wave : wave - C::NSX) * 256 + 4 * lane;   // first dword of the lane in its part
    const int u = q / R;                            // step of the group
    const ScaleSrc& S = isx ? xs : ws;
    const uint32_t r = S.row0 + (uint32_t)(q % R);
    P.s_step = S.rows * 4u;
    P.s_base = r * 4u + (uint32_t)u * P.s_step;
  }
}

// Global -> LDS copies of stage `st` (elements [64 st, 64 st + 64)) into slot
// `sb`.  A 16-byte chunk (16 elements, or 32 packed e2m1) is loaded iff it
// lies inside [lo, hi); others -- and every chunk of a stage wholly outside,
// e.g. a prefetch past the last stage -- read as zeros without touching memory.
template <class C>
__device__ __forceinline__ void issue_stage(uint8_t* sb, const Operand& X, const Operand& W,
                                            const Plan<C>& P, int st, int lo, int hi) {
  const int wave = wave_id();
  const int kk = st * BKS;
  constexpr int WE = C::F4 ? 32 : 16;              // elements per W chunk
  constexpr int WR = C::F4 ? 32 : 16;              // W rows per copy
  const int xlo = lo - kk <= 0 ? 0 : (lo - kk + 15) / 16;
  const int xhi = hi - kk <= 0 ? 0 : (hi - kk) / 16;
  const int wlo = lo - kk <= 0 ? 0 : (lo - kk + WE - 1) / WE;
  const int whi = hi - kk <= 0 ? 0 : (hi - kk) / WE;
  const int xc = (int)(P.xoff >> 28), wc = (int)(P.woff >> 28);
  const uint32_t xo = (xc >= xlo && xc < xhi) ? (P.xoff & 0x0fffffffu) : kOOB;
  const uint32_t wo = (wc >= wlo && wc < whi) ? (P.woff & 0x0fffffffu) : kOOB;
#pragma unroll
  for (int i = 0; i < C::QX; ++i) {
    const int q = wave * C::QX + i;
    const uint32_t so = ((uint32_t)st * C::XROW << X.pl) + (uint32_t)(q * 16) * X.ld;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(X.data, (lds_ptr_t)(sb + q * 1024), 16, xo, so, 0, 0);
  }
  uint8_t* wb = sb + C::XBYTES;
#pragma unroll
  for (int i = 0; i < C::QW; ++i) {
    const int q = wave * C::QW + i;
    const uint32_t so = ((uint32_t)st * C::WROW << W.pl) + (uint32_t)(q * WR) * W.ld;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(W.data, (lds_ptr_t)(wb + q * 1024), 16, wo, so, 0, 0);
  }
}

// 16 bytes per lane global -> LDS at LDS byte address `lds` when `go` != 0.
// The branch lives inside the asm statement, so the loop body stays a single
// basic block for the compiler (a branch there costs the register allocator
// dearly); M0 is saved and restored around the copy.  The copy is not known to
// the compiler: callers order it with explicit vmcnt waits.
__device__ __forceinline__ void dma16_if(int go, __amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t saved;
  asm volatile(
      "s_cmp_eq_u32 %1, 0\n\t"
      "s_cbranch_scc1 1f\n\t"
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %4, 0 offen lds\n\t"
      "s_mov_b32 m0, %0\n"
      "1:"
      : "=&s"(saved)
      : "s"(go), "v"(voff), "s"(lds), "s"(rsrc)
      : "memory", "scc");
#endif
}

// dma16_if with a scalar byte offset `soff` added to the address.
__device__ __forceinline__ void dma16_if_so(int go, __amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff,
                                            uint32_t lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  uint32_t saved;
  asm volatile(
      "s_cmp_eq_u32 %1, 0\n\t"
      "s_cbranch_scc1 1f\n\t"
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %4, %5 offen lds\n\t"
      "s_mov_b32 m0, %0\n"
      "1:"
      : "=&s"(saved)
      : "s"(go), "v"(voff), "s"(lds), "s"(rsrc), "s"(soff)
      : "memory", "scc");
#endif
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(lds_ptr_t)(const_cast<void*>(p));
}

// Scale group of steps tg .. tg+GSTEPS-1 into scale slot `ss` (ssr: the
// scale buffer of the wave's operand).  Step-major: waves w < NSD copy 1 KB
// each; plain: every wave copies SPW pieces of 32 rows (tg a multiple of 8).
template <class C>
__device__ __forceinline__ void issue_scales(uint8_t* ss, __amdgpu_buffer_rsrc_t ssr, const Plan<C>& P,
                                             int tg, bool live) {
  const int wave = wave_id();
  if constexpr (C::PS) {
    const int go = uniform(live ? 1 : 0);
    const uint32_t v = P.s_base + (uint32_t)tg * 4u;
#pragma unroll
    for (int i = 0; i < C::SPW; ++i)
      dma16_if_so(go, ssr, v, (uint32_t)uniform((int)(P.s_step * (uint32_t)i)), lds_addr(ss + (wave * C::SPW + i) * 1024));
  } else {
    const int go = (live && wave < C::NSD) ? 1 : 0;
    dma16_if(uniform(go), ssr, P.s_base + (uint32_t)tg * P.s_step, lds_addr(ss + wave * 1024));
  }
}

// Plain scales: piece i (rows 32 (w SPW + i) .. +31 of the slot) of the group
// of steps tg .. tg+7 into scale slot `ss`, when `live` (wave-uniform i).
template <class C>
__device__ __forceinline__ void issue_scale_piece(uint8_t* ss, __amdgpu_buffer_rsrc_t ssr, const Plan<C>& P,
                                                  int tg, int i, bool live) {
  static_assert(C::PS, "plain scales");
  const int wave = wave_id();
  dma16_if_so(uniform(live ? 1 : 0), ssr, P.s_base + (uint32_t)tg * 4u, (uint32_t)uniform((int)(P.s_step * (uint32_t)i)),
              lds_addr(ss + (wave * C::SPW + i) * 1024));
}

// Fragments and raw scale dwords of the stage in data slot `sb`, whose step is
// step u of the group held in scale slot `ss`.
template <class C>
__device__ __forceinline__ void read_stage(const uint8_t* sb, const uint8_t* ss, int u, Frags<C>& F,
                                           uint32_t (&xs)[C::FM], uint32_t (&ws)[C::FN]) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int hsel = lane >> 5;
  const int r32 = lane & 31;
  const int sw = swz4(r32);
  const int c0 = hsel ^ sw;            // elements 16 hsel .. +15
  const int c1 = (2 + hsel) ^ sw;      // elements 32 + 16 hsel .. +15
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
    if constexpr (C::F4) {
      // 32 packed fp4 values, elements 32 hsel .. +31: one 16-byte chunk
      v4i lo = *reinterpret_cast<const v4i*>(row + (hsel ^ swz2(r32)) * 16);
      F.a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], 0, 0, 0, 0};
    } else {
      v4i lo = *reinterpret_cast<const v4i*>(row + c0 * 16);
      v4i hi = *reinterpret_cast<const v4i*>(row + c1 * 16);
      F.a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }
  if constexpr (C::PS) {
    // slot row m: 8 dwords, half (u / 4) ^ ((m >> 3) & 1) holding steps 4 (u / 4) ..
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(ss);
    const int d = ((((u >> 2) ^ (r32 >> 3)) & 1) << 2) | (u & 3);
#pragma unroll
    for (int i = 0; i < C::FM; ++i) xs[i] = s32[(wm * C::WTM + i * 32 + r32) * 8 + d];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) ws[j] = s32[(C::BM + wn * C::WTN + j * 32 + r32) * 8 + d];
  } else {
    const uint32_t* sx = reinterpret_cast<const uint32_t*>(ss) + u * C::BM;
    const uint32_t* sy = reinterpret_cast<const uint32_t*>(ss) + C::GSTEPS * C::BM + u * C::BN;
#pragma unroll
    for (int i = 0; i < C::FM; ++i) xs[i] = sx[wm * C::WTM + i * 32 + r32];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) ws[j] = sy[wn * C::WTN + j * 32 + r32];
  }
}

// Move the scale byte of the lane's 32-element block of stage st (block
// 2 st + hsel: byte 2 (st & 1) + hsel of the step's dword) to byte 0, where
// op_sel 0 reads it; blocks wholly outside [lo, hi) get the neutral scale
// 127, so zero-filled data never meets a NaN scale byte.  A block that only
// partly overlaps [lo, hi) (a bound that is not a multiple of 32) keeps its
// scale: its in-range elements are real data.
template <class C>
__device__ __forceinline__ void finish_scales(uint32_t (&xs)[C::FM], uint32_t (&ws)[C::FN], int st, int lo,
                                              int hi) {
  const int hsel = (threadIdx.x % kWave) >> 5;
  const int sh = 8 * hsel + 16 * (st & 1);
  const int k = st * BKS + 32 * hsel;
  const bool out = k + 32 <= lo || k >= hi;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) xs[i] = out ? 127u : (xs[i] >> sh);
#pragma unroll
  for (int j = 0; j < C::FN; ++j) ws[j] = out ? 127u : (ws[j] >> sh);
}

// MFMAs B .. E-1 of a stage (fragment t: row block t / FN, column block
// t % FN).  FIRST: the reduction's first stage, which starts each accumulator
// from zero (the MFMA's C operand) instead of reading it.
template <class C, int B, int E, bool FIRST = false>
__device__ __forceinline__ void mfma_range(const Frags<C>& F, const uint32_t (&xs)[C::FM],
                                           const uint32_t (&ws)[C::FN], v16f (&acc)[C::FM][C::FN]) {
#pragma unroll
  for (int t = B; t < E; ++t) {
    const int i = t / C::FN, j = t % C::FN;
    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(F.a[j], F.b[i], FIRST ? (v16f){} : acc[i][j], C::WFMT,
                                                                 MXGG_FMT_E4M3, 0, (int)ws[j], 0, (int)xs[i]);
  }
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

#define MXGG_WAIT_VM(n) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory")
#define MXGG_BARRIER() asm volatile("s_barrier" ::: "memory")
#define MXGG_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// Scheduling recipe: NM MFMAs with the ND DS reads spread over the first NMD
// of them and the NV VMEM issues (LDS-DMA copies) over the rest, so every read
// is issued before any copy.
template <int I, int NM, int NMD, int ND, int NV>
__device__ __forceinline__ void interleave_step() {
  if constexpr (I < NM) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                  // 1 MFMA
    if constexpr (I < NMD) {
      constexpr int d = (ND * (I + 1)) / NMD - (ND * I) / NMD;
      if constexpr (d > 0) __builtin_amdgcn_sched_group_barrier(0x100, d, 0);   // DS reads
    } else {
      constexpr int J = I - NMD, NR = NM - NMD;
      constexpr int v = (NV * (J + 1)) / NR - (NV * J) / NR;
      if constexpr (v > 0) __builtin_amdgcn_sched_group_barrier(0x010, v, 0);   // VMEM
    }
    interleave_step<I + 1, NM, NMD, ND, NV>();
  }
}

// One stage: multiply stage s0 + r (Fc, xc, wc), read stage s0 + r + 1 into
// (Fn, xn, wn), start the copies of stage s0 + r + NS and, when stage
// s0 + r + 1 opens a scale group, the scales of the group after it.
// (s0 is the ring's first stage, even, in slot 0; t0 = s0 / 2 its step.)
// FIRST: stage s0, whose MFMAs start the accumulators from zero.  TAIL:
// kStageFull as described; kStageNoCopy2 / 1 / 0, the fourth, third and
// second stage from the end, start no copies (any would fetch a stage past the
// run: zero fills that only load the LDS port), so the wait for the next
// stage allows for the copies of 2 / 1 / 0 later stages only; kStageLast,
// the last stage, only multiplies.
constexpr int kStageFull = 0, kStageNoCopy2 = 1, kStageNoCopy1 = 2, kStageNoCopy0 = 3, kStageLast = 4;
template <class C, bool FIRST = false, int TAIL = kStageFull>
__device__ __forceinline__ void ring_stage(uint8_t* smem, const Operand& X, const Operand& W,
                                           __amdgpu_buffer_rsrc_t ssr, const Plan<C>& P, int s0, int r,
                                           int lo, int hi, Frags<C>& Fc, uint32_t (&xc)[C::FM],
                                           uint32_t (&wc)[C::FN], Frags<C>& Fn, uint32_t (&xn)[C::FM],
                                           uint32_t (&wn)[C::FN], v16f (&acc)[C::FM][C::FN]) {
  constexpr int NMMA = C::FM * C::FN;
  constexpr int NE = NMMA >= 8 ? 2 : 1;       // MFMAs issued ahead of the barrier
  constexpr int NDS = C::FM * 2 + (C::F4 ? C::FN : C::FN * 2) + C::FM + C::FN;
  const int rn = r + 1;
  uint8_t* cur = smem + (r % C::NS) * C::STAGE;
  const uint8_t* nxt = smem + (rn % C::NS) * C::STAGE;
  // scale groups: GSTAGES stages each, counted from the ring's first stage
  // (step-major) or from the 8-step piece holding it (plain: g0 stages into
  // it; its first step tb a multiple of 8)
  const int g0 = C::PS ? (s0 & (C::GSTAGES - 1)) : 0;
  const int gr = g0 + rn;
  const uint8_t* snx = smem + C::SOFF + ((gr / C::GSTAGES) & 1) * C::SSLOT;
  if constexpr (TAIL == kStageLast) {
    mfma_range<C, 0, NMMA, FIRST>(Fc, xc, wc, acc);
    hold(Fc, xc, wc);
    MXGG_SCHED_FENCE();
    return;
  }
  mfma_range<C, 0, NE, FIRST>(Fc, xc, wc, acc);
  MXGG_SCHED_FENCE();
  // this wave's copies of stage r+1 have landed (the copies of the NS-2
  // stages after it may still be in flight; in the tail, of those issued)
  if constexpr (TAIL == kStageNoCopy1)
    MXGG_WAIT_VM(C::LPS);
  else if constexpr (TAIL == kStageNoCopy0)
    MXGG_WAIT_VM(0);
  else
    MXGG_WAIT_VM((C::NS - 2) * C::LPS);
  MXGG_BARRIER();                           // ... every wave's; and stage r's slot is free
  MXGG_SCHED_FENCE();
  // LDS reads first, then the copies: a read issued after an LDS-DMA load
  // may otherwise be given the load's offset register as its destination
  // while the load still uses it.
  read_stage<C>(nxt, snx, (gr / 2) % C::GSTEPS, Fn, xn, wn);
  // stage r+1 opening scale group g = gr / GSTAGES frees the slot of group g-1
  // (last read, of stage r, before this barrier): group g+1 goes there
  // (a group that starts past the reduction range is never read: not copied,
  // so the drain after the last stage waits for no memory read)
  if constexpr (TAIL == kStageFull) {
    const int tg = (s0 - g0) / 2 + (gr / C::GSTAGES + 1) * C::GSTEPS;
    uint8_t* sn = smem + C::SOFF + ((gr / C::GSTAGES + 1) & 1) * C::SSLOT;
    if constexpr (C::PS) {
      // plain: the group's SPW pieces one per stage over its first SPW
      // stages (a burst of copies stalls the waves' issue); a group whose
      // later pieces would fall on the copy-free last stages starts at or
      // past the last stage, so it is never read (and tg * STEP >= hi)
      const int gs = gr % C::GSTAGES;
      issue_scale_piece<C>(sn, ssr, P, tg, gs < C::SPW ? gs : 0, gs < C::SPW && tg * STEP < hi);
    } else {
      const bool opens = gr % C::GSTAGES == 0 && tg * STEP < hi;
      issue_scales<C>(sn, ssr, P, tg, opens);
    }
    issue_stage<C>(cur, X, W, P, s0 + r + C::NS, lo, hi);
  }
  mfma_range<C, NE, NMMA, FIRST>(Fc, xc, wc, acc);
  interleave_step<0, NMMA - NE, (NMMA - NE) / 2, NDS, TAIL == kStageFull ? C::LPS : 0>();
  static_assert(C::NS == 4, "the tail stages assume a 4-deep ring");
  MXGG_SCHED_FENCE();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  finish_scales<C>(xn, wn, s0 + rn, lo, hi);
  // keep the current set allocated past the rewrite of the next one
  hold(Fc, xc, wc);
  MXGG_SCHED_FENCE();
}

template <class C>
__device__ __forceinline__ void zero_acc(v16f (&acc)[C::FM][C::FN]) {
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) acc[i][j] = (v16f){};
}

// ---------------------------------------------------------------------------
// Main loop with X in two-stage slots (XLine).  Stage r of the run (stage
// s0 + r, s0 even) issues the copies of W stage r + 3 into W slot r % 3 and
// of half (r + 1) & 1 of X pair q = (r + 5) / 2 (stages 2q, 2q+1) into X slot
// q % 3, the slot of pair (r - 1) / 2, whose stages the waves have read by
// the stage's barrier; the prologue copies pairs 0 and 1, half 0 of pair 2 and
// W stages 0 .. 2.  Every full stage thus issues QX + QW copies, and the wait
// before reading stage r + 1 (W copies two stages earlier, X copies three or
// more) allows the previous stage's copies in flight.
// ---------------------------------------------------------------------------

// Half h of the X copies of the pair whose first stage is st (even) into X
// slot xb; the chunk bounds as in issue_stage.
template <class C>
__device__ __forceinline__ void issue_xhalf(uint8_t* xb, const Operand& X, const Plan<C>& P, int st, int h,
                                            int lo, int hi) {
  const int wave = wave_id();
  const int kk = st * BKS;
  const int xlo = lo - kk <= 0 ? 0 : (lo - kk + 15) / 16;
  const int xhi = hi - kk <= 0 ? 0 : (hi - kk) / 16;
  const int ue = (int)(P.xoff >> 28), uo = (int)(P.xoff2 >> 28);
  const uint32_t xe = (ue >= xlo && ue < xhi) ? (P.xoff & 0x0fffffffu) : kOOB;
  const uint32_t xo = (uo >= xlo && uo < xhi) ? (P.xoff2 & 0x0fffffffu) : kOOB;
  const int c0 = (wave * 2 + h) * C::QX;   // first copy (even)
#pragma unroll
  for (int i = 0; i < C::QX; ++i) {
    const uint32_t so = ((uint32_t)st * C::XROW << X.pl) + (uint32_t)((c0 + i) * 8) * X.ld;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(X.data, (lds_ptr_t)(xb + (c0 + i) * 1024), 16, (i & 1) ? xo : xe, so,
                                             0, 0);
  }
}

// W copies of stage st into W slot wb (issue_stage's W part, e4m3).
template <class C>
__device__ __forceinline__ void issue_wstage(uint8_t* wb, const Operand& W, const Plan<C>& P, int st, int lo,
                                             int hi) {
  const int wave = wave_id();
  const int kk = st * BKS;
  const int wlo = lo - kk <= 0 ? 0 : (lo - kk + 15) / 16;
  const int whi = hi - kk <= 0 ? 0 : (hi - kk) / 16;
  const int wc = (int)(P.woff >> 28);
  const uint32_t wo = (wc >= wlo && wc < whi) ? (P.woff & 0x0fffffffu) : kOOB;
#pragma unroll
  for (int i = 0; i < C::QW; ++i) {
    const int q = wave * C::QW + i;
    const uint32_t so = ((uint32_t)st * C::WROW << W.pl) + (uint32_t)(q * 16) * W.ld;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(W.data, (lds_ptr_t)(wb + q * 1024), 16, wo, so, 0, 0);
  }
}

// read_stage for two-stage X slots: the stage of parity h2 of X slot xb, the
// W stage in wb, step u of the scale group in ss.
template <class C>
__device__ __forceinline__ void read_stage_xd(const uint8_t* xb, const uint8_t* wb, const uint8_t* ss, int u, int h2,
                                              Frags<C>& F, uint32_t (&xs)[C::FM], uint32_t (&ws)[C::FN]) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int hsel = lane >> 5;
  const int r32 = lane & 31;
  const int g = (r32 & 7) ^ ((r32 >> 3) & 1);
  const int x0 = ((h2 << 2) | hsel) ^ g;        // elements 16 hsel .. +15
  const int x1 = ((h2 << 2) | 2 | hsel) ^ g;    // elements 32 + 16 hsel .. +15
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const uint8_t* row = xb + (wm * C::WTM + i * 32 + r32) * 128;
    v4i lo = *reinterpret_cast<const v4i*>(row + x0 * 16);
    v4i hi = *reinterpret_cast<const v4i*>(row + x1 * 16);
    F.b[i] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  const int sw = swz4(r32);
  const int c0 = hsel ^ sw;
  const int c1 = (2 + hsel) ^ sw;
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const uint8_t* row = wb + (wn * C::WTN + j * 32 + r32) * C::WROW;
    v4i lo = *reinterpret_cast<const v4i*>(row + c0 * 16);
    v4i hi = *reinterpret_cast<const v4i*>(row + c1 * 16);
    F.a[j] = (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  const uint32_t* sx = reinterpret_cast<const uint32_t*>(ss) + u * C::BM;
  const uint32_t* sy = reinterpret_cast<const uint32_t*>(ss) + C::GSTEPS * C::BM + u * C::BN;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) xs[i] = sx[wm * C::WTM + i * 32 + r32];
#pragma unroll
  for (int j = 0; j < C::FN; ++j) ws[j] = sy[wn * C::WTN + j * 32 + r32];
}

// One stage of the two-stage-X ring, as ring_stage: multiply stage s0 + r,
// read stage s0 + r + 1, issue the copies described above.  TAIL: kXdFull;
// kXdNoCopy1 / kXdNoCopy0, the third and second stage from the end, issue
// nothing and wait for the copies of one / no later stage; kXdLast only
// multiplies.
constexpr int kXdFull = 0, kXdNoCopy1 = 1, kXdNoCopy0 = 2, kXdLast = 3;
template <class C, bool FIRST = false, int TAIL = kXdFull>
__device__ __forceinline__ void ring_stage_xd(uint8_t* smem, const Operand& X, const Operand& W,
                                              __amdgpu_buffer_rsrc_t ssr, const Plan<C>& P, int s0, int r,
                                              int lo, int hi, Frags<C>& Fc, uint32_t (&xc)[C::FM],
                                              uint32_t (&wc)[C::FN], Frags<C>& Fn, uint32_t (&xn)[C::FM],
                                              uint32_t (&wn)[C::FN], v16f (&acc)[C::FM][C::FN]) {
  constexpr int NMMA = C::FM * C::FN;
  constexpr int NE = NMMA >= 8 ? 2 : 1;
  constexpr int NDS = C::FM * 2 + C::FN * 2 + C::FM + C::FN;
  const int rn = r + 1;
  const uint8_t* xnx = smem + ((rn >> 1) % C::NS) * C::XSLOT;
  const uint8_t* wnx = smem + C::WOFF + (rn % C::NS) * C::WBYTES;
  const uint8_t* snx = smem + C::SOFF + ((rn / C::GSTAGES) & 1) * C::SSLOT;
  if constexpr (TAIL == kXdLast) {
    mfma_range<C, 0, NMMA, FIRST>(Fc, xc, wc, acc);
    hold(Fc, xc, wc);
    MXGG_SCHED_FENCE();
    return;
  }
  mfma_range<C, 0, NE, FIRST>(Fc, xc, wc, acc);
  MXGG_SCHED_FENCE();
  if constexpr (TAIL == kXdNoCopy0)
    MXGG_WAIT_VM(0);
  else
    MXGG_WAIT_VM(C::LPS);
  MXGG_BARRIER();
  MXGG_SCHED_FENCE();
  read_stage_xd<C>(xnx, wnx, snx, (rn / 2) % C::GSTEPS, rn & 1, Fn, xn, wn);
  if constexpr (TAIL == kXdFull) {
    const int tg = s0 / 2 + (rn / C::GSTAGES + 1) * C::GSTEPS;
    uint8_t* sn = smem + C::SOFF + ((rn / C::GSTAGES + 1) & 1) * C::SSLOT;
    issue_scales<C>(sn, ssr, P, tg, rn % C::GSTAGES == 0 && tg * STEP < hi);
    const int q = (r + 5) >> 1;
    issue_xhalf<C>(smem + (q % C::NS) * C::XSLOT, X, P, s0 + 2 * q, (r + 1) & 1, lo, hi);
    issue_wstage<C>(smem + C::WOFF + (r % C::NS) * C::WBYTES, W, P, s0 + r + 3, lo, hi);
  }
  mfma_range<C, NE, NMMA, FIRST>(Fc, xc, wc, acc);
  interleave_step<0, NMMA - NE, (NMMA - NE) / 2, NDS, TAIL == kXdFull ? C::LPS : 0>();
  MXGG_SCHED_FENCE();
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  finish_scales<C>(xn, wn, s0 + rn, lo, hi);
  hold(Fc, xc, wc);
  MXGG_SCHED_FENCE();
}

// ring_mainloop for two-stage X slots (the same range, padding and ZSTART
// meaning; a run of n stages runs n rounded up to even, at least 6).
template <class C, bool ZSTART>
__device__ __forceinline__ void ring_mainloop_xd(uint8_t* smem, const Operand& X, const Operand& W,
                                                 const ScaleSrc& xss, const ScaleSrc& wss, int s0, int s1,
                                                 int lo, int hi, v16f (&acc)[C::FM][C::FN]) {
  if (s0 >= s1) s1 = s0 + 1;
  s0 &= ~1;
  Plan<C> P;
  make_plan<C>(P, X, W, xss, wss);
  const __amdgpu_buffer_rsrc_t ssr = wave_id() < C::NSX ? xss.rsrc : wss.rsrc;
  issue_scales<C>(smem + C::SOFF, ssr, P, s0 / 2, true);
  issue_scales<C>(smem + C::SOFF + C::SSLOT, ssr, P, s0 / 2 + C::GSTEPS, true);
  issue_xhalf<C>(smem, X, P, s0, 0, lo, hi);
  issue_xhalf<C>(smem, X, P, s0, 1, lo, hi);
  issue_wstage<C>(smem + C::WOFF, W, P, s0, lo, hi);
  issue_xhalf<C>(smem + C::XSLOT, X, P, s0 + 2, 0, lo, hi);
  issue_xhalf<C>(smem + C::XSLOT, X, P, s0 + 2, 1, lo, hi);
  issue_wstage<C>(smem + C::WOFF + C::WBYTES, W, P, s0 + 1, lo, hi);
  issue_xhalf<C>(smem + 2 * C::XSLOT, X, P, s0 + 4, 0, lo, hi);
  issue_wstage<C>(smem + C::WOFF + 2 * C::WBYTES, W, P, s0 + 2, lo, hi);
  MXGG_WAIT_VM(3 * C::QX + 2 * C::QW);   // pair 0 and W stage 0 (and the scales before them)
  MXGG_BARRIER();
  Frags<C> Fa, Fb;
  uint32_t xa[C::FM], wa[C::FN], xb[C::FM], wb[C::FN];
  read_stage_xd<C>(smem, smem + C::WOFF, smem + C::SOFF, 0, 0, Fa, xa, wa);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  finish_scales<C>(xa, wa, s0, lo, hi);
  const int n = s1 - s0;
  const int nr = n < 6 ? 6 : (n + 1) & ~1;
  ring_stage_xd<C, ZSTART>(smem, X, W, ssr, P, s0, 0, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
#pragma nounroll
  for (int r = 1; r < nr - 3; r += 2) {
    ring_stage_xd<C>(smem, X, W, ssr, P, s0, r, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
    ring_stage_xd<C>(smem, X, W, ssr, P, s0, r + 1, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
  }
  ring_stage_xd<C, false, kXdNoCopy1>(smem, X, W, ssr, P, s0, nr - 3, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
  ring_stage_xd<C, false, kXdNoCopy0>(smem, X, W, ssr, P, s0, nr - 2, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
  ring_stage_xd<C, false, kXdLast>(smem, X, W, ssr, P, s0, nr - 1, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
  MXGG_WAIT_VM(0);
}

// Reduction over the 64-element stages [s0, s1) restricted to the element
// range [lo, hi) (chunks and scale blocks outside it are zero / neutral),
// into acc.  ZSTART: the first stage's MFMAs start from zero, so acc needs no
// clearing (256 accumulator writes per lane, which the compiler otherwise puts
// between the tile set-up and the first copies, twice over when an empty range
// has a path of its own); else the caller zeroes acc.  An empty range runs one
// stage wholly outside [lo, hi).
// The ring starts at the even stage s0 & ~1 so that scale groups cover whole
// steps; an odd stage count runs one stage past s1.  Those extra stages are
// wholly outside [lo, hi): zero data, neutral scales, exactly zero added.
template <class C, bool ZSTART = true>
__device__ __forceinline__ void ring_mainloop(uint8_t* smem, const Operand& X, const Operand& W,
                                              const ScaleSrc& xss, const ScaleSrc& wss, int s0, int s1,
                                              int lo, int hi, v16f (&acc)[C::FM][C::FN]) {
  if constexpr (C::XD) {
    ring_mainloop_xd<C, ZSTART>(smem, X, W, xss, wss, s0, s1, lo, hi, acc);
  } else {
    if (s0 >= s1) s1 = s0 + 1;
    s0 &= ~1;
    Plan<C> P;
    make_plan<C>(P, X, W, xss, wss);
    // the scale buffer this wave copies from (wave-uniform)
    const __amdgpu_buffer_rsrc_t ssr = wave_id() < (C::PS ? C::NXW : C::NSX) ? xss.rsrc : wss.rsrc;
    // scale groups 0 and 1, then stages s0 .. s0+NS-1 (scales first: every
    // wait for a stage's copies then covers the scale copies issued before it)
    const int g0 = C::PS ? (s0 & (C::GSTAGES - 1)) : 0;
    const int tb = (s0 - g0) / 2;
    issue_scales<C>(smem + C::SOFF, ssr, P, tb, true);
    issue_scales<C>(smem + C::SOFF + C::SSLOT, ssr, P, tb + C::GSTEPS, true);
  #pragma unroll
    for (int i = 0; i < C::NS; ++i) issue_stage<C>(smem + i * C::STAGE, X, W, P, s0 + i, lo, hi);
    MXGG_WAIT_VM((C::NS - 1) * C::LPS);
    MXGG_BARRIER();
    Frags<C> Fa, Fb;
    uint32_t xa[C::FM], wa[C::FN], xb[C::FM], wb[C::FN];
    read_stage<C>(smem, smem + C::SOFF, g0 / 2, Fa, xa, wa);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    finish_scales<C>(xa, wa, s0, lo, hi);
    const int n = s1 - s0;
    if constexpr (ZSTART) {
      // stages run: n rounded up to even, at least 6 (those past s1 hold
      // zeros); the last four start no copies (the prologue and the full
      // stages already issued every stage of the run), the last reads nothing
      const int nr = n < 6 ? 6 : (n + 1) & ~1;
      ring_stage<C, true>(smem, X, W, ssr, P, s0, 0, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
      ring_stage<C>(smem, X, W, ssr, P, s0, 1, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
  #pragma nounroll
      for (int r = 2; r < nr - 4; r += 2) {
        ring_stage<C>(smem, X, W, ssr, P, s0, r, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
        ring_stage<C>(smem, X, W, ssr, P, s0, r + 1, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
      }
      ring_stage<C, false, kStageNoCopy2>(smem, X, W, ssr, P, s0, nr - 4, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
      ring_stage<C, false, kStageNoCopy1>(smem, X, W, ssr, P, s0, nr - 3, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
      ring_stage<C, false, kStageNoCopy0>(smem, X, W, ssr, P, s0, nr - 2, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
      ring_stage<C, false, kStageLast>(smem, X, W, ssr, P, s0, nr - 1, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
    } else {
  #pragma nounroll
      for (int r = 0; r < n; r += 2) {
        ring_stage<C>(smem, X, W, ssr, P, s0, r, lo, hi, Fa, xa, wa, Fb, xb, wb, acc);
        ring_stage<C>(smem, X, W, ssr, P, s0, r + 1, lo, hi, Fb, xb, wb, Fa, xa, wa, acc);
      }
    }
    // copies past the last stage (zero fills, scale groups) may still be
    // writing LDS: drain them before the LDS is reused or released
    MXGG_WAIT_VM(0);
  }
}

// The in-range elements of the 16-element chunk at cs (a multiple of 16)
// that straddles a bound of the reduction range [lo, hi).  The ring copies
// whole chunks only, so a bound that is not a multiple of 16 leaves these
// out; they are added here as one more 64-element MFMA step whose fragments
// are loaded into registers, every element outside [lo, hi) and every other
// chunk of the step zero.  MFMA operand layout (the one read_stage builds):
// lane half h holds elements 16h .. 16h+15 of the step in dwords 0-3 and
// 32+16h .. 32+16h+15 in dwords 4-7, and supplies the scale of the step's
// block h (elements 32h .. 32h+31).  e4m3 on both sides (the weight
// gradient's operands).
template <class C>
__device__ __forceinline__ void edge_chunk(const Operand& X, const Operand& W, const ScaleSrc& xss,
                                           const ScaleSrc& wss, int cs, int lo, int hi,
                                           v16f (&acc)[C::FM][C::FN]) {
  static_assert(!C::F4 && !C::PS, "edge chunks: e4m3 operands, step-major scales only");
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int h = lane >> 5, r32 = lane & 31;
  const int kb = cs & ~(BKS - 1);                  // the step holding the chunk
  const int ci = (cs - kb) >> 4;                   // chunk of the step: half (ci & 1), dwords 4 (ci >> 1) ..
  const bool mine = h == (ci & 1);
  // bytes b of the chunk with lo <= cs + b < hi
  uint32_t mk[4];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    uint32_t m = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int k = cs + 4 * d + b;
      m |= (k >= lo && k < hi) ? (0xffu << (8 * b)) : 0u;
    }
    mk[d] = mine ? m : 0u;
  }
  Frags<C> F;
  uint32_t xs[C::FM], ws[C::FN];
  const int t = kb / STEP;
  const int blk = (kb / 32 + h) & 3;               // byte of the lane's block in the step's dword
  const bool live = kb + 32 * h < hi && kb + 32 * h + 32 > lo;
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const uint32_t row = (uint32_t)(wm * C::WTM + i * 32 + r32);
    const v4i v =
        __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(X.data, operand_off(X, row, (uint32_t)cs), 0, 0));
    v8i f = (v8i){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int w = v[d] & (int)mk[d];
      if (ci >> 1) f[4 + d] = w; else f[d] = w;
    }
    F.b[i] = f;
    const uint32_t s = __builtin_amdgcn_raw_buffer_load_b32(xss.rsrc, ((uint32_t)t * xss.rows + xss.row0 + row) * 4u, 0, 0);
    xs[i] = live ? (s >> (8 * blk)) & 0xffu : 127u;
  }
#pragma unroll
  for (int j = 0; j < C::FN; ++j) {
    const uint32_t row = (uint32_t)(wn * C::WTN + j * 32 + r32);
    const v4i v =
        __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(W.data, operand_off(W, row, (uint32_t)cs), 0, 0));
    v8i f = (v8i){0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int w = v[d] & (int)mk[d];
      if (ci >> 1) f[4 + d] = w; else f[d] = w;
    }
    F.a[j] = f;
    const uint32_t s = __builtin_amdgcn_raw_buffer_load_b32(wss.rsrc, ((uint32_t)t * wss.rows + wss.row0 + row) * 4u, 0, 0);
    ws[j] = live ? (s >> (8 * blk)) & 0xffu : 127u;
  }
  mfma_range<C, 0, C::FM * C::FN>(F, xs, ws, acc);
  hold(F, xs, ws);
  // What follows (a second edge step, the epilogue) may reuse these operand
  // registers at once; the compiler does not count the scale operands as
  // in-flight MFMA reads, so give the last MFMA time to read them.
#if defined(__HIP_DEVICE_COMPILE__)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#endif
}

// Edge chunks of [lo, hi) (see edge_chunk): the chunk holding lo when lo is
// not a multiple of 16, and the one holding hi when hi is not (once when
// they are the same chunk).
template <class C>
__device__ __forceinline__ void edge_chunks(const Operand& X, const Operand& W, const ScaleSrc& xss,
                                            const ScaleSrc& wss, int lo, int hi, v16f (&acc)[C::FM][C::FN]) {
  if (hi <= lo) return;
  const int clo = lo & ~15, chi = hi & ~15;
  if (lo & 15) edge_chunk<C>(X, W, xss, wss, clo, lo, hi, acc);
  if ((hi & 15) && !((lo & 15) && chi == clo)) edge_chunk<C>(X, W, xss, wss, chi, lo, hi, acc);
}

// Store 4 consecutive output columns c .. c+3 of row r (those below `cols`)
// of a row-major output of element type out_dtype.  vec: rows and `out`
// aligned for one 16-byte (f32) or 8-byte (16-bit) store of the four.
// BF16_ONLY: round to bf16 first whatever the output type (wgrad semantics).
template <bool BF16_ONLY>
__device__ __forceinline__ void store4(uint8_t* out, int64_t ldo, int out_dtype, bool vec, int r, int c,
                                       int cols, float v0, float v1, float v2, float v3) {
  // f32 and f16 outputs of BF16_ONLY hold the bf16-rounded value (f16:
  // converted from it)
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
      if (BF16_ONLY) {
        v0 = round_bf16(v0); v1 = round_bf16(v1); v2 = round_bf16(v2); v3 = round_bf16(v3);
      }
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

__device__ __forceinline__ bool store4_vec(const uint8_t* out, int64_t ldo, int out_dtype) {
  return out_dtype == MXGG_DTYPE_F32 ? ((ldo % 4) == 0 && ((uintptr_t)out % 16) == 0)
                                     : ((ldo % 4) == 0 && ((uintptr_t)out % 8) == 0);
}

// Store an accumulator tile.  Lane l of fragment (i, j) holds output row
// wm*WTM + 32i + l%32 and columns wn*WTN + 32j + 8(q/4) + 4(l/32) + q%4.
template <class C, bool BF16_ONLY>
__device__ __forceinline__ void store_tile(const v16f (&acc)[C::FM][C::FN], uint8_t* out,
                                           int64_t ldo, int rows, int cols, int out_dtype) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const bool vec = store4_vec(out, ldo, out_dtype);
#pragma unroll
  for (int i = 0; i < C::FM; ++i) {
    const int r = wm * C::WTM + i * 32 + (lane & 31);
    if (r >= rows) continue;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int c = wn * C::WTN + j * 32 + 8 * q4 + 4 * (lane >> 5);
        store4<BF16_ONLY>(out, ldo, out_dtype, vec, r, c, cols, acc[i][j][4 * q4 + 0], acc[i][j][4 * q4 + 1],
                          acc[i][j][4 * q4 + 2], acc[i][j][4 * q4 + 3]);
      }
    }
  }
}

// fp32 partial tile of a split unit, in accumulator-register order: values
// 4q .. 4q+3 of lane l of fragment f = (wave * FM + i) * FN + j are the float4
// at index (f * 4 + q) * 64 + l of the unit's BM x BN slot, so every store
// instruction writes one contiguous 1 KB run.  (With a lane's 16 values
// contiguous instead, each instruction scatters 64 16-byte pieces over 4 KB
// and the partial store takes about four times as long.)
template <class C>
__device__ __forceinline__ void store_partial(const v16f (&acc)[C::FM][C::FN], float* slot) {
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
#pragma unroll
  for (int i = 0; i < C::FM; ++i)
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
      float4* d = reinterpret_cast<float4*>(slot) + (int64_t)((wave * C::FM + i) * C::FN + j) * 4 * kWave + lane;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        d[q * kWave] =
            make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
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

// BF16: the 16-bit output type (bf16, else f16), fixed at compile time so the
// staging loop carries no per-write type test.  RB16 (f16 only): convert the
// bf16-rounded value (the weight gradient's store semantics).
template <class C, bool BF16, bool RB16 = false>
__device__ __forceinline__ void store_tile_lds(const v16f (&acc)[C::FM][C::FN], uint8_t* smem,
                                               uint8_t* out, int64_t ldo, int rows, int cols) {
  constexpr int RB = C::WTN * 2;                 // staged row bytes
  constexpr int NCH = RB / 16;                   // 16-byte chunks per row
  constexpr int AVAIL = C::LDS / C::NW;           // LDS bytes per wave
  constexpr int FPP = store_pass_rows(C::FM, AVAIL / (32 * RB));   // fragment rows per pass
  static_assert(FPP >= 1 && C::FM % FPP == 0, "store staging");
  static_assert(64 % NCH == 0, "store row width");
  const int wave = wave_id();
  const int lane = threadIdx.x % kWave;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  uint8_t* area = smem + wave * (FPP * 32 * RB);
  // a wave's rows and columns all inside the output: no per-store checks
  const bool whole = (wm + 1) * C::WTM <= rows && (wn + 1) * C::WTN <= cols;
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
          if constexpr (BF16) {
            w0 = pack_bf16x2(a[4 * q4 + 0], a[4 * q4 + 1]);
            w1 = pack_bf16x2(a[4 * q4 + 2], a[4 * q4 + 3]);
          } else {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            float f0 = a[4 * q4 + 0], f1 = a[4 * q4 + 1], f2 = a[4 * q4 + 2], f3 = a[4 * q4 + 3];
            if constexpr (RB16) {
              f0 = round_bf16(f0); f1 = round_bf16(f1); f2 = round_bf16(f2); f3 = round_bf16(f3);
            }
            h2 x = {(_Float16)f0, (_Float16)f1};
            h2 y = {(_Float16)f2, (_Float16)f3};
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
    if (whole) {
      // Non-temporal stores: the kernel never reads its output back, while
      // its operand copies depend on L2 hits (same-box A/B over the 36-shape
      // sweep: forward +0.6%, wgrad +1.3% geomean, up to +4% on E=8 wgrad).
#pragma unroll
      for (int it = 0; it < FPP * 32 / RPI; ++it) {
        const int r = it * RPI + lane / NCH;
        const int c = lane % NCH;
        const v4i v = *reinterpret_cast<const v4i*>(area + r * RB + ((c ^ (r % NCH)) * 16));
        const int row = wm * C::WTM + i0 * 32 + r;
        const int col = wn * C::WTN + c * 8;
        __builtin_nontemporal_store(v, reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(out) + (int64_t)row * ldo + col));
      }
    } else {
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
}

// ---------------------------------------------------------------------------
// scale re-layout: plain (rows, nblk) e8m0 scales -> [batch][step][row] dwords
// ---------------------------------------------------------------------------

// One operand's scales: `batches` blocks of `rows` rows (row r of batch b at
// src + b * ld_b + r * ld_r), nblk = K/32 bytes per row.  Output dword
// (b, t, r) at dst[(b * steps + t) * rows + r] holds bytes 4t .. 4t+3 of the
// row; bytes past nblk are 127 (2**0), so a partial last step needs no
// masking in the GEMM.
struct ScaleJob {
  const uint8_t* src; int64_t ld_r; int64_t ld_b;
  uint32_t* dst; int rows; int batches; int nblk; int steps;
  int tiles_r; int tiles_t;      // 64-row x 16-step tiles per batch
};

// An e4m3 operand copied from rows into row pairs (the layout the GEMM
// copies in whole 128-byte lines): `batches` blocks of `rows` rows (even) of
// `len` bytes, row r of batch b at src + b * ld_b + r * ld_r (16-byte
// aligned); byte k of row r of batch b goes to dst + b * rows * ld_dst +
// (r / 2) * 2 * ld_dst + (k / 64) * 128 + (r % 2) * 64 + k % 64, ld_dst =
// len rounded up to 64, bytes past len zero.
struct PairJob {
  const uint8_t* src; int64_t ld_r; int64_t ld_b;
  uint8_t* dst; int ld_dst; int pairs; int batches; int len;   // pairs = rows / 2
};

struct ScaleJobs {
  ScaleJob j[2];
  int tiles0;                    // workgroups of job 0 (job 1 follows)
  int tiles01;                   // workgroups of jobs 0 and 1 (pair job d follows)
  PairJob d;
  int tiles_d;                   // workgroups of pair job d (pair job d2 follows)
  PairJob d2;
};

// Pair job, workgroup w: row pair q of batch b (w = b * pairs + q), its
// 2 * ld_dst output bytes in 16-byte chunks, consecutive threads on
// consecutive chunks (coalesced stores; four threads read one 64-byte row
// piece).  The source is read once: non-temporal loads.
__device__ __forceinline__ void pair_chunks(const PairJob& J, int w) {
  const int b = w / J.pairs, q = w - b * J.pairs;
  const uint8_t* src = J.src + b * J.ld_b + (int64_t)(2 * q) * J.ld_r;
  uint8_t* dst = J.dst + ((int64_t)b * J.pairs + q) * 2 * J.ld_dst;
  for (int o = 16 * (int)threadIdx.x; o < 2 * J.ld_dst; o += 16 * 256) {
    const int h = (o >> 6) & 1, k = (o >> 7) * 64 + (o & 63);
    v4i v = {0, 0, 0, 0};
    if (k < J.len) v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(src + h * J.ld_r + k));
    *reinterpret_cast<v4i*>(dst + o) = v;
  }
}

// 64 rows x 16 steps per workgroup (256 threads): each thread reads 16
// source bytes of one row (4 steps; one 16-byte load when the chunk is
// aligned and inside the row), the tile is transposed through LDS, and each
// thread writes the dwords of 4 consecutive rows for one step (one 16-byte
// store when aligned and inside the operand).
__global__ __launch_bounds__(256) void scale_relayout_kernel(ScaleJobs js) {
  __shared__ uint32_t tile[16][65];
  int bid = blockIdx.x;
  if (bid >= js.tiles01) {
    bid -= js.tiles01;
    if (bid < js.tiles_d)
      pair_chunks(js.d, bid);
    else
      pair_chunks(js.d2, bid - js.tiles_d);
    return;
  }
  const int which = bid < js.tiles0 ? 0 : 1;
  const ScaleJob& J = js.j[which];
  if (which) bid -= js.tiles0;
  const int per_batch = J.tiles_r * J.tiles_t;
  const int b = bid / per_batch;
  const int rt = (bid % per_batch) % J.tiles_r;
  const int tt = (bid % per_batch) / J.tiles_r;
  const int r0 = rt * 64, t0 = tt * 16;
  {
    const int r = r0 + threadIdx.x / 4;
    const int tq = threadIdx.x % 4;                // steps t0 + 4 tq .. + 3
    const int blk0 = 4 * t0 + 16 * tq;             // first scale byte of the chunk
    uint32_t v[4] = {0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu, 0x7f7f7f7fu};
    if (r < J.rows && blk0 < J.nblk) {
      const uint8_t* src = J.src + (int64_t)b * J.ld_b + (int64_t)r * J.ld_r + blk0;
      if (blk0 + 16 <= J.nblk && ((uintptr_t)src & 15) == 0) {
        const uint4 q = *(const uint4*)src;
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
      } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          uint32_t w = 0;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int i = 4 * s + q;
            const uint32_t byte = blk0 + i < J.nblk ? (uint32_t)src[i] : 127u;
            w |= byte << (8 * q);
          }
          v[s] = w;
        }
      }
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) tile[4 * tq + s][threadIdx.x / 4] = v[s];
  }
  __syncthreads();
  {
    const int ts = threadIdx.x / 16;               // step of the tile
    const int rq = threadIdx.x % 16;               // rows 4 rq .. 4 rq + 3
    const int t = t0 + ts;
    const int r = r0 + 4 * rq;
    if (t < J.steps && r < J.rows) {
      uint32_t* out = J.dst + ((int64_t)b * J.steps + t) * J.rows + r;
      if (r + 4 <= J.rows && ((uintptr_t)out & 15) == 0) {
        *(uint4*)out = make_uint4(tile[ts][4 * rq], tile[ts][4 * rq + 1], tile[ts][4 * rq + 2],
                                  tile[ts][4 * rq + 3]);
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (r + q < J.rows) out[q] = tile[ts][4 * rq + q];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// forward / dgrad
// ---------------------------------------------------------------------------

struct FwdParams {
  const uint8_t* a; int64_t lda;
  const uint8_t* b; int64_t ldb_n; int64_t ldb_e;
  // A scales: step-major [T][M] dwords (T = cdiv(K, 128)), or (plain-scale
  // kernels, Cfg::PS) to_mx's (M, K/32) bytes with row stride as_ld; B
  // scales: step-major [E][T][N] dwords, or plain (E, N, K/32) with row
  // stride bs_ld.  as_bytes / bs_expert: bytes of A's / of one expert's scales.
  const uint8_t* as; uint32_t as_bytes;
  const uint8_t* bs; uint32_t bs_expert;
  const int32_t* offs; int E; int64_t M; int64_t N; int64_t K;
  uint8_t* out; int out_dtype; int64_t ldo;
  int grid_n; int group_m; int xcd;
  float* part; int par; int slots;          // split: partial slots, resident workgroups, slot count
  int quads;                                // last round as 128 x 128 quarter tiles (quad_dp)
  int a_pl; int b_pl;                       // operand layouts: 0 rows, 1 row pairs, 2 row quads (Operand)
  uint32_t as_ld; uint32_t bs_ld;           // plain scales: bytes per row (multiples of 16)
};

// Epilogue of the whole-tile kernels, fixed at compile time so that the
// common case carries none of the others' register pressure (with every
// variant in one kernel the allocator spilled accumulators to scratch and
// reloaded them serially in the epilogue): kEpiBf16 / kEpiF16 are bf16 / f16
// outputs whose rows are 16-byte aligned (row stride a multiple of 8
// elements, 16-byte aligned base), staged through LDS; kEpiF32 stores f32
// directly, and kEpiBf16Any / kEpiF16Any 16-bit rows off the 16-byte grid;
// kEpiAny (the wgrad's other outputs) picks the type per call.
constexpr int kEpiAny = 0, kEpiBf16 = 1, kEpiF16 = 2, kEpiF32 = 3, kEpiBf16Any = 4, kEpiF16Any = 5;

// Epilogue of a whole-tile launch for this output (host side).
inline int pick_epi(int out_dtype, int64_t ldo, const void* out) {
  const bool al16 = ldo % 8 == 0 && (uintptr_t)out % 16 == 0;
  if (al16 && out_dtype == MXGG_DTYPE_BF16) return kEpiBf16;
  if (al16 && out_dtype == MXGG_DTYPE_F16) return kEpiF16;
  if (out_dtype == MXGG_DTYPE_F32) return kEpiF32;
  return out_dtype == MXGG_DTYPE_BF16 ? kEpiBf16Any : kEpiF16Any;
}

struct FwdTile {
  int expert;
  int64_t row0; int rows;     // output rows row0 .. row0 + rows - 1 (one group)
  int64_t n0; int cols;       // output columns n0 .. n0 + cols - 1
};

// Tile of logical index lt (0 <= lt < tiles) after the XCD swizzle and the
// expert-aligned band order (route_tile: bands of at most GROUP_M m-blocks
// inside one group); false when it holds no output rows.  Wave-uniform.
// wg: the groups as load_groups read them when E <= 64 (else offs is read).
template <class C>
__device__ __forceinline__ bool fwd_tile(const FwdParams& p, int lt, int tiles, const WaveGroups& wg,
                                         FwdTile& tl) {
  const int t = p.xcd > 1 ? xcd_swizzle(lt, tiles, p.xcd) : lt;
  int pn;
  const TileRoute r = p.E <= kWave ? route_tile(wg, p.E, C::BM, p.grid_n, p.group_m, t, pn)
                                   : route_tile(p.offs, p.E, C::BM, p.grid_n, p.group_m, t, pn);
  if (r.expert < 0) return false;
  tl.expert = r.expert;
  tl.row0 = (int64_t)r.start + (int64_t)r.block * C::BM;
  int64_t rows64 = p.M - tl.row0;
  if (rows64 > r.rows) rows64 = r.rows;
  if (rows64 <= 0) return false;
  tl.rows = (int)rows64;
  tl.n0 = (int64_t)pn * C::BN;
  tl.cols = (int)(p.N - tl.n0 < C::BN ? p.N - tl.n0 : C::BN);
  return true;
}

// Tiles of a 256 x 256 launch computed whole when its last round runs as
// 128 x 128 quarter tiles (fwd_quad_kernel): a reduction too short to split
// (fewer than kMinSplitTotal steps), at most kSplitMaxRounds full rounds
// before it, and four quarters per tile of the rem = T % P tiles fit one
// round.  A lone round of 256 x 256 tiles at K = 2048 takes about as long as
// a full round (42 us against 38; the copies of one tile per CU are latency
// bound), its quarters on four times the CUs about 60% of that.
__host__ __device__ inline int quad_dp(int T, int P) {
  if (T <= 0 || P <= 0 || T / P > kSplitMaxRounds) return T;
  const int rem = T % P;
  return rem > 0 && 4 * rem <= P ? T - rem : T;
}

template <class C>
__device__ __forceinline__ Split fwd_split(const FwdParams& p, int tiles) {
  if (p.quads) return Split{quad_dp(tiles, p.par), 1, 0};
  return split_plan(tiles, p.par, (int)((p.K + STEP - 1) / STEP), p.slots, C::BM * C::BN * 4 / 1024);
}

// Tile tl whole (PIECES = false; epilogue EPI), or piece `piece` of S of it
// into partial slot `slot` (PIECES = true).
template <class C, bool PIECES, int EPI>
__device__ __forceinline__ void fwd_tile_run(const FwdParams& p, uint8_t* smem, const FwdTile& tl, int piece, int S,
                                             int slot) {
  const int64_t row0 = tl.row0, n0 = tl.n0;
  const int rows = tl.rows, cols = tl.cols;

  const Operand X = make_operand(p.a, p.lda, p.a_pl, row0, rows);
  const Operand W = make_operand(p.b + (int64_t)tl.expert * p.ldb_e, p.ldb_n, p.b_pl, n0, cols);
  const ScaleSrc xs{make_rsrc(p.as, p.as_bytes), C::PS ? p.as_ld : (uint32_t)p.M, (uint32_t)row0};
  const ScaleSrc ws{make_rsrc(p.bs + (int64_t)tl.expert * p.bs_expert, p.bs_expert), C::PS ? p.bs_ld : (uint32_t)p.N,
                    (uint32_t)n0};

  v16f acc[C::FM][C::FN];   // set by ring_mainloop
  const int K = (int)p.K;
  if constexpr (PIECES) {
    int a, b;
    split_range(0, (int)((p.K + STEP - 1) / STEP), piece, S, a, b);
    const int lo = STEP * a;
    const int hi = STEP * b < K ? STEP * b : K;
    ring_mainloop<C>(smem, X, W, xs, ws, lo / BKS, (hi + BKS - 1) / BKS, lo, hi, acc);
    store_partial<C>(acc, p.part + (int64_t)slot * (C::BM * C::BN));
  } else {
    // the f32 epilogue's register allocation spills when the first stage is
    // peeled: it keeps the accumulators zeroed up front
    if constexpr (EPI == kEpiF32) {
      zero_acc<C>(acc);
      ring_mainloop<C, false>(smem, X, W, xs, ws, 0, (K + BKS - 1) / BKS, 0, K, acc);
    } else {
      ring_mainloop<C>(smem, X, W, xs, ws, 0, (K + BKS - 1) / BKS, 0, K, acc);
    }
    if constexpr (EPI == kEpiBf16) {
      store_tile_lds<C, true>(acc, smem, p.out + (row0 * p.ldo + n0) * 2, p.ldo, rows, cols);
    } else if constexpr (EPI == kEpiF16) {
      store_tile_lds<C, false>(acc, smem, p.out + (row0 * p.ldo + n0) * 2, p.ldo, rows, cols);
    } else if constexpr (EPI == kEpiF32) {
      store_tile<C, false>(acc, p.out + (row0 * p.ldo + n0) * 4, p.ldo, rows, cols, MXGG_DTYPE_F32);
    } else {
      static_assert(EPI == kEpiBf16Any || EPI == kEpiF16Any, "forward epilogue");
      store_tile<C, false>(acc, p.out + (row0 * p.ldo + n0) * 2, p.ldo, rows, cols,
                           EPI == kEpiBf16Any ? MXGG_DTYPE_BF16 : MXGG_DTYPE_F16);
    }
  }
}

// Tile of logical index lt, run as fwd_tile_run describes.
template <class C, bool PIECES, int EPI>
__device__ __forceinline__ void fwd_run(const FwdParams& p, uint8_t* smem, int lt, int piece, int S, int slot,
                                        int tiles, const WaveGroups& wg) {
  FwdTile tl;
  if (fwd_tile<C>(p, lt, tiles, wg, tl)) fwd_tile_run<C, PIECES, EPI>(p, smem, tl, piece, S, slot);
}

// Groups of a forward launch and its m-block count: one read of offs when
// E <= 64 (kept for the tile lookup), else a scan of offs in 64-group chunks.
template <class C>
__device__ __forceinline__ int fwd_groups(const FwdParams& p, WaveGroups& wg) {
  if (p.E <= kWave) {
    wg = load_groups(p.offs, p.E, C::BM);
    return wg.total;
  }
  wg = WaveGroups{0, 0, 0, 0, 0};
  return route_total(p.offs, p.E, C::BM);
}

// PIECES = false: workgroup i < dp computes tile i whole (epilogue EPI).
// PIECES = true: workgroup u < units computes piece u % S of tile dp + u / S
// into partial slot u.  Other workgroups exit.  (Two kernels rather than one
// with both paths: sharing a register allocation slows the whole-tile loop by
// ~2%.)
template <class C, bool PIECES, int EPI = kEpiBf16>
__global__ __launch_bounds__(C::NT) void fwd_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS];
  WaveGroups wg;
  const int tiles = fwd_groups<C>(p, wg) * p.grid_n;
  const Split sp = fwd_split<C>(p, tiles);
  const int pid = blockIdx.x;
  if constexpr (PIECES) {
    if (pid < sp.units) fwd_run<C, true, kEpiAny>(p, smem, sp.dp + pid / sp.S, pid % sp.S, sp.S, pid, tiles, wg);
  } else {
    if (pid < sp.dp) fwd_run<C, false, EPI>(p, smem, pid, 0, 1, 0, tiles, wg);
  }
}

// The last round of a launch of C tiles (256 x 256) as Q tiles (128 x 128):
// workgroup u < 4 * (tiles - dp) computes quarter u % 4 (row half u / 2 % 2,
// column half u % 2) of tile dp + u / 4, clipped to the tile; the routing and
// the plan are C's, so the whole-tile kernel and this one agree on dp.
template <class C, class Q, int EPI>
__global__ __launch_bounds__(Q::NT) void fwd_quad_kernel(FwdParams p) {
  static_assert(C::BM == 2 * Q::BM && C::BN == 2 * Q::BN && C::WFMT == Q::WFMT, "quarter tiles");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Q::LDS];
  WaveGroups wg;
  const int tiles = fwd_groups<C>(p, wg) * p.grid_n;
  const Split sp = fwd_split<C>(p, tiles);
  if (sp.units) return;   // a last round split into pieces is not quartered
  const int dp = sp.dp;
  const int u = blockIdx.x;
  if (u >= 4 * (tiles - dp)) return;
  FwdTile tl;
  if (!fwd_tile<C>(p, dp + u / 4, tiles, wg, tl)) return;
  const int dr = (u & 2) ? Q::BM : 0, dc = (u & 1) ? Q::BN : 0;
  if (tl.rows <= dr || tl.cols <= dc) return;
  tl.row0 += dr;
  tl.rows = tl.rows - dr < Q::BM ? tl.rows - dr : Q::BM;
  tl.n0 += dc;
  tl.cols = tl.cols - dc < Q::BN ? tl.cols - dc : Q::BN;
  fwd_tile_run<Q, false, EPI>(p, smem, tl, 0, 1, 0);
}

// Sum over the S pieces (slots base + s * BM * BN, s = 0 .. S-1, in that
// order) of the 16 partial values of lane `lane` of fragment f.
template <class C>
__device__ __forceinline__ void sum_pieces(const float* base, int S, int f, int lane, float (&v)[16]) {
#pragma unroll
  for (int q = 0; q < 16; ++q) v[q] = 0.f;
  const float4* src = reinterpret_cast<const float4*>(base) + (int64_t)f * 4 * kWave + lane;
  for (int s = 0; s < S; ++s) {
    const float4* x = src + (int64_t)s * (C::BM * C::BN / 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = x[q * kWave];
      v[4 * q] += t.x; v[4 * q + 1] += t.y; v[4 * q + 2] += t.z; v[4 * q + 3] += t.w;
    }
  }
}

// Store the 16 values of lane `lane` of fragment f of a tile (rows x cols at
// `out`, row stride ldo).
template <class C, bool BF16_ONLY>
__device__ __forceinline__ void store_fragment_lane(const float (&v)[16], int f, int lane, uint8_t* out,
                                                    int64_t ldo, int rows, int cols, int out_dtype) {
  const int wave = f / (C::FM * C::FN), i = (f / C::FN) % C::FM, j = f % C::FN;
  const int wm = wave / C::WGN, wn = wave % C::WGN;
  const int r = wm * C::WTM + i * 32 + (lane & 31);
  if (r >= rows) return;
  const bool vec = store4_vec(out, ldo, out_dtype);
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    const int c = wn * C::WTN + j * 32 + 8 * q4 + 4 * (lane >> 5);
    store4<BF16_ONLY>(out, ldo, out_dtype, vec, r, c, cols, v[4 * q4], v[4 * q4 + 1], v[4 * q4 + 2], v[4 * q4 + 3]);
  }
}

// Fragments per tile and reduce items per tile (4 fragments, one per wave of
// a 256-thread workgroup).
template <class C>
struct ReduceShape {
  static constexpr int NF = C::NW * C::FM * C::FN;
  static constexpr int CH = NF / 4;
  static_assert(NF % 4 == 0, "reduce items");
};

// Store one reduce item: fragments 4c .. 4c+3 of a tile, fragment f = 4c +
// wave of the workgroup, with FN = 4 the column blocks j = 0 .. 3 of row
// block i of wave tile wt, i.e. 32 rows x WTN columns.  16-bit outputs with
// 16-byte aligned rows whose block lies wholly inside the tile go through LDS
// (store_item_lds), so that each global store writes 4 whole row segments of
// WTN * 2 bytes; the per-lane stores (store_fragment_lane) write 16 bytes of
// each of 32 rows instead, and serve every other output and tiles of other
// wave shapes (FN != 4).  Every wave of the workgroup calls it for the same
// item: the LDS path holds workgroup barriers, and its condition is the same
// for the four fragments.
template <class C, bool BF16_ONLY>
__device__ __forceinline__ void store_item_lds(const float (&v)[16], int f, int lane, uint8_t* out, int64_t ldo,
                                               int rows, int cols, int out_dtype, uint8_t* blk) {
  constexpr int RB = C::WTN * 2;                 // staged row bytes
  constexpr int NCH = RB / 16;                   // 16-byte chunks per row (XOR-swizzled by row in blk)
  constexpr int RPI = 64 / NCH;                  // rows per store instruction
  constexpr int RPW = 32 / C::NW;                // rows each wave stores
  static_assert(NCH <= 64 && 64 % NCH == 0 && RPW % RPI == 0, "reduce block shape");
  const int wt = f / (C::FM * C::FN), i = (f / C::FN) % C::FM, j = f % C::FN;
  const int r0 = (wt / C::WGN) * C::WTM + i * 32, c0 = (wt % C::WGN) * C::WTN;
  const bool staged = out_dtype != MXGG_DTYPE_F32 && ldo % 8 == 0 && (uintptr_t)out % 16 == 0 &&
                      r0 + 32 <= rows && c0 + C::WTN <= cols;
  if (!staged) {
    store_fragment_lane<C, BF16_ONLY>(v, f, lane, out, ldo, rows, cols, out_dtype);
    return;
  }
  const int m = lane & 31, h = lane >> 5;
  __syncthreads();                               // the previous item's reads of blk are done
#pragma unroll
  for (int q4 = 0; q4 < 4; ++q4) {
    uint32_t w0, w1;
    if (out_dtype == MXGG_DTYPE_BF16) {
      w0 = pack_bf16x2(v[4 * q4], v[4 * q4 + 1]);
      w1 = pack_bf16x2(v[4 * q4 + 2], v[4 * q4 + 3]);
    } else {
      float f0 = v[4 * q4], f1 = v[4 * q4 + 1], f2 = v[4 * q4 + 2], f3 = v[4 * q4 + 3];
      if (BF16_ONLY) {
        f0 = round_bf16(f0); f1 = round_bf16(f1); f2 = round_bf16(f2); f3 = round_bf16(f3);
      }
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      h2 x = {(_Float16)f0, (_Float16)f1}, y = {(_Float16)f2, (_Float16)f3};
      w0 = __builtin_bit_cast(uint32_t, x);
      w1 = __builtin_bit_cast(uint32_t, y);
    }
    const int c = 4 * j + q4;                    // 16-byte chunk (8 columns) of the block row
    *reinterpret_cast<uint2*>(blk + m * RB + ((c ^ (m % NCH)) * 16) + 8 * h) = make_uint2(w0, w1);
  }
  __syncthreads();
  const int wid = wave_id();
#pragma unroll
  for (int it = 0; it < RPW / RPI; ++it) {       // wave wid: rows RPW wid .. RPW wid + RPW - 1
    const int r = wid * RPW + it * RPI + lane / NCH;
    const int c = lane % NCH;
    const v4i val = *reinterpret_cast<const v4i*>(blk + r * RB + ((c ^ (r % NCH)) * 16));
    __builtin_nontemporal_store(
        val, reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(out) + (int64_t)(r0 + r) * ldo + c0 + c * 8));
  }
}

template <class C, bool BF16_ONLY>
__device__ __forceinline__ void store_item(const float (&v)[16], int f, int lane, uint8_t* out, int64_t ldo,
                                           int rows, int cols, int out_dtype, uint8_t* blk) {
  if constexpr (C::FN == 4 && C::NW == 4)
    store_item_lds<C, BF16_ONLY>(v, f, lane, out, ldo, rows, cols, out_dtype, blk);
  else
    store_fragment_lane<C, BF16_ONLY>(v, f, lane, out, ldo, rows, cols, out_dtype);
}

// Split tiles of a forward launch: item (v, c) = fragments 4c .. 4c+3 of split
// tile v, summed over its pieces and stored.  The plan is recomputed from
// offs exactly as fwd_kernel computed it.
template <class C>
__global__ __launch_bounds__(256) void fwd_reduce_kernel(FwdParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t blk[32 * C::WTN * 2];
  WaveGroups wg;
  const int tiles = fwd_groups<C>(p, wg) * p.grid_n;
  const Split sp = fwd_split<C>(p, tiles);
  if (sp.units == 0) return;
  constexpr int CH = ReduceShape<C>::CH;
  const int rem = sp.units / sp.S;
  const int lane = threadIdx.x % kWave;
  const int esz = p.out_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  for (int item = blockIdx.x; item < rem * CH; item += gridDim.x) {
    const int v = item / CH, f = (item % CH) * 4 + wave_id();
    FwdTile tl;
    if (!fwd_tile<C>(p, sp.dp + v, tiles, wg, tl)) continue;
    float acc[16];
    sum_pieces<C>(p.part + (int64_t)v * sp.S * (C::BM * C::BN), sp.S, f, lane, acc);
    store_item<C, false>(acc, f, lane, p.out + (tl.row0 * p.ldo + tl.n0) * esz, p.ldo, tl.rows, tl.cols,
                         p.out_dtype, blk);
  }
}

// ---------------------------------------------------------------------------
// weight gradient: one workgroup per (group, N tile, K tile); the group's
// token range is the reduction range (masked at unaligned ends).
// ---------------------------------------------------------------------------

struct WgradParams {
  const uint8_t* go; int64_t ld_go;
  const uint8_t* ia; int64_t ld_ia;
  const uint8_t* gs; uint32_t gs_bytes;     // GO scales, step-major [T][N] dwords (T = cdiv(M, 128))
  const uint8_t* is; uint32_t is_bytes;     // IA scales, step-major [T][K] dwords
  const int32_t* offs; int E; int64_t M; int64_t N; int64_t K;
  uint8_t* out; int out_dtype;
  int tiles_n; int tiles_k;
  float* part; int dp; int S; int units;    // split plan (host): see split_plan
  int dev; int par; int slots;              // dev: plan on the device (wgrad_groups / wgrad_plan) from par, slots
  int go_pl; int ia_pl;                     // operand layouts: 0 rows, 1 row pairs (Operand)
};

struct WgradTile {
  int g;                      // group
  int64_t n0; int rows;       // output rows (n) n0 .. n0 + rows - 1
  int64_t k0; int cols;       // output columns (k) k0 .. k0 + cols - 1
};

template <class C>
__device__ __forceinline__ WgradTile wgrad_tile(const WgradParams& p, int lt) {
  WgradTile t;
  const int per = p.tiles_n * p.tiles_k;
  t.g = lt / per;
  const int x = lt % per;
  t.n0 = (int64_t)(x / p.tiles_k) * C::BM;   // X side: rows of go_t
  t.k0 = (int64_t)(x % p.tiles_k) * C::BN;   // W side: rows of ia_t
  t.rows = (int)(p.N - t.n0 < C::BM ? p.N - t.n0 : C::BM);
  t.cols = (int)(p.K - t.k0 < C::BN ? p.K - t.k0 : C::BN);
  return t;
}

// Reduction steps (of STEP elements) the longest group touches.  Wave-uniform.
__device__ __forceinline__ int wgrad_max_steps(const int32_t* __restrict__ offs, int E, int64_t M) {
  const int lane = threadIdx.x & (kWave - 1);
  int m = 0;
  for (int base = 0; base < E; base += kWave) {
    const int e = base + lane;
    int n = 0;
    if (e < E) {
      int lo = e > 0 ? offs[e - 1] : 0;
      int hi = offs[e];
      if (lo < 0) lo = 0;
      if (hi > M) hi = (int)M;
      n = hi > lo ? (hi + STEP - 1) / STEP - lo / STEP : 0;
    }
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int o = __shfl_xor(n, d, kWave);
      n = o > n ? o : n;
    }
    m = uniform(n) > m ? uniform(n) : m;
  }
  return m;
}

// Split plan of a wgrad launch: the host's (dev = 0), or, for a lone
// under-filled round of several groups (dev = 1), one made here from the
// longest group, which sets the round's length (the host sees only the
// average).  Every kernel of the launch computes the same plan.
template <class C>
__device__ __forceinline__ Split wgrad_plan(const WgradParams& p) {
  if (!p.dev) return Split{p.dp, p.S, p.units};
  const int tiles = p.E * p.tiles_n * p.tiles_k;
  return split_plan(tiles, p.par, wgrad_max_steps(p.offs, p.E, p.M), p.slots, C::BM * C::BN * 4 / 1024);
}

__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int o = __shfl_xor(v, d, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// Per-group split of a lone wgrad round (dev = 1, E <= 64).  Groups differ in
// length, and one piece count for every tile leaves the round as long as the
// longest group's pieces while short groups' tiles idle.  Greedy
// apportionment instead: from one piece per tile, the first group with the
// longest pieces gets one more piece per tile, again and again, while the
// units (E * TNK tiles' pieces, TNK = tiles_n * tiles_k) fit the budget
// min(par, slots), every piece keeps kMinSplitSteps steps and no tile exceeds
// kMaxSplit pieces.  Each candidate is priced with split_plan's cost model,
// the round lasting as long as its longest piece; the best one is kept if it
// saves kSplitMinGainNs, else no tile is split.  Integer, lane-parallel and
// deterministic: every workgroup of every kernel of the launch gets the same
// plan.  Lane g < E holds group g's entries.
struct WgradGroups {
  int s;       // pieces per tile of group `lane` (1: whole, as one piece); 0 past E
  int c0;      // first unit of group `lane`'s tiles (exclusive prefix of TNK * s)
  int units;   // units in all; 0: no tile is split
};

template <class C>
__device__ __forceinline__ WgradGroups wgrad_groups(const WgradParams& p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int tnk = p.tiles_n * p.tiles_k;
  int n = 0;
  if (lane < p.E) {
    int lo = lane > 0 ? p.offs[lane - 1] : 0;
    int hi = p.offs[lane];
    if (lo < 0) lo = 0;
    if (hi > p.M) hi = (int)p.M;
    n = hi > lo ? (hi + STEP - 1) / STEP - lo / STEP : 0;
    if (n > (1 << 20)) n = 1 << 20;   // keeps the cost model's products in int32
  }
  int s = lane < p.E ? 1 : 0, len = n, units = p.E * tnk, best_s = s, best_units = 0;
  const int budget = p.par < p.slots ? p.par : p.slots;
  const int len0 = wave_max(len);
  const int tail = (int)kTailNsPerStep * len0;
  int best = (int)kSplitMinGainNs;
  constexpr int kib = C::BM * C::BN * 4 / 1024;
  if (len0 >= kMinSplitTotal) {
    for (int it = 0; it < kWave && units + tnk <= budget; ++it) {
      const int m = wave_max(len);
      const int g = __builtin_ctzll(__ballot(lane < p.E && len == m));
      const int gn = lane_value(n, g), gs = lane_value(s, g);
      if (gs >= kMaxSplit || gn / (gs + 1) < kMinSplitSteps) break;
      if (lane == g) {
        s = gs + 1;
        len = (n + s - 1) / s;
      }
      units += tnk;
      const int gain = tail - (int)kTailNsPerStep * wave_max(len) - (int)kSplitFixedNs -
                       units * kib * (int)kSplitNsPerMiB / 1024;
      if (gain > best) {
        best = gain;
        best_s = s;
        best_units = units;
      }
    }
  }
  WgradGroups w;
  w.units = best_units;
  w.s = lane < p.E ? (best_units ? best_s : 1) : 0;
  w.c0 = wave_incl_scan(tnk * w.s) - tnk * w.s;
  return w;
}

// Tiles below the returned index run whole (PIECES = false).
template <class C>
__device__ __forceinline__ int wgrad_whole(const WgradParams& p) {
  if (p.dev && p.E <= kWave) return wgrad_groups<C>(p).units ? 0 : p.E * p.tiles_n * p.tiles_k;
  return wgrad_plan<C>(p).dp;
}

// Tile, piece and piece count of unit u of the piece kernel; false past the
// plan's units.  Unit u writes partial slot u; a tile's pieces are
// consecutive units.
template <class C>
__device__ __forceinline__ bool wgrad_unit(const WgradParams& p, int u, int& lt, int& piece, int& S) {
  if (p.dev && p.E <= kWave) {
    const WgradGroups w = wgrad_groups<C>(p);
    if (u >= w.units) return false;
    const int tnk = p.tiles_n * p.tiles_k;
    const int g = __builtin_ctzll(__ballot(w.s > 0 && w.c0 + tnk * w.s > u));
    S = lane_value(w.s, g);
    const int r = u - lane_value(w.c0, g);
    lt = g * tnk + r / S;
    piece = r % S;
    return true;
  }
  const Split sp = wgrad_plan<C>(p);
  if (u >= sp.units) return false;
  lt = sp.dp + u / sp.S;
  piece = u % sp.S;
  S = sp.S;
  return true;
}

// Split tile v of the reduce kernel: its tile, first partial slot and piece
// count; false past the split tiles.
template <class C>
__device__ __forceinline__ bool wgrad_split_tile(const WgradParams& p, int v, int& lt, int& base, int& S) {
  if (p.dev && p.E <= kWave) {
    const WgradGroups w = wgrad_groups<C>(p);
    const int tnk = p.tiles_n * p.tiles_k;
    if (!w.units || v >= p.E * tnk) return false;
    const int g = v / tnk;
    S = lane_value(w.s, g);
    base = lane_value(w.c0, g) + (v - g * tnk) * S;
    lt = v;
    return true;
  }
  const Split sp = wgrad_plan<C>(p);
  if (sp.S < 2 || v >= sp.units / sp.S) return false;
  lt = sp.dp + v;
  base = v * sp.S;
  S = sp.S;
  return true;
}

// Group of dispatch slot y of the whole-tile grid: the groups longest first
// (most reduction steps; ties by index).  The hardware starts workgroups in
// blockIdx order as CUs free up, so with more tiles than CUs this is the
// longest-processing-time-first schedule: a long group's tiles start in the
// first round instead of behind short groups (E=8, N=K=2048 with groups of 3
// to 44 steps: a 44-step tile then bounds the launch, not a short round plus
// a 36-step one).  Which workgroup computes a tile never changes its result.
// E <= 64 (one lane per group); past that, index order.
__device__ __forceinline__ int wgrad_slot_group(const WgradParams& p, int y) {
  if (p.E > kWave || p.E == 1) return y;
  const int lane = threadIdx.x & (kWave - 1);
  int n = -1;
  if (lane < p.E) {
    int lo = lane > 0 ? p.offs[lane - 1] : 0;
    int hi = p.offs[lane];
    if (lo < 0) lo = 0;
    if (hi > p.M) hi = (int)p.M;
    n = hi > lo ? (hi + STEP - 1) / STEP - lo / STEP : 0;
  }
  int rank = 0;
  for (int g = 0; g < p.E; ++g) {
    const int v = lane_value(n, g);
    rank += (v > n || (v == n && g < lane)) ? 1 : 0;
  }
  return __ffsll((long long)__ballot(lane < p.E && rank == y)) - 1;
}

// PIECES = false: grid (tiles_n * tiles_k, E), workgroup (x, y) computes tile
// g * tiles_n * tiles_k + x of group g = wgrad_slot_group(y) whole when below
// wgrad_whole (epilogue EPI); true: workgroup u computes the piece
// wgrad_unit assigns it.
template <class C, bool PIECES, int EPI = kEpiAny>
__global__ __launch_bounds__(C::NT) void wgrad_kernel(WgradParams p) {
  __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS];
  int lt, piece = 0, S = 1;
  if constexpr (PIECES) {
    if (!wgrad_unit<C>(p, (int)blockIdx.x, lt, piece, S)) return;
  } else {
    // (wgrad_whole is every tile or none except for E = 1 or E > 64, where
    // slots map to groups in index order)
    lt = wgrad_slot_group(p, (int)blockIdx.y) * p.tiles_n * p.tiles_k + (int)blockIdx.x;
    if (lt >= wgrad_whole<C>(p)) return;
  }
  const WgradTile tl = wgrad_tile<C>(p, lt);
  const int g = tl.g;
  const int64_t n0 = tl.n0, k0 = tl.k0;
  const int rows = tl.rows, cols = tl.cols;
  int lo = g > 0 ? p.offs[g - 1] : 0;
  int hi = p.offs[g];
  if (lo < 0) lo = 0;
  if (hi > p.M) hi = (int)p.M;
  if (PIECES && hi > lo) {
    // piece of the group's steps lo/STEP .. cdiv(hi, STEP)-1, clipped to [lo, hi)
    const int a0 = lo / STEP;
    int a, b;
    split_range(a0, (hi + STEP - 1) / STEP - a0, piece, S, a, b);
    if (STEP * a > lo) lo = STEP * a;
    if (STEP * b < hi) hi = STEP * b;
  }

  const Operand X = make_operand(p.go, p.ld_go, p.go_pl, n0, rows);
  const Operand W = make_operand(p.ia, p.ld_ia, p.ia_pl, k0, cols);
  const ScaleSrc xs{make_rsrc(p.gs, p.gs_bytes), (uint32_t)p.N, (uint32_t)n0};
  const ScaleSrc ws{make_rsrc(p.is, p.is_bytes), (uint32_t)p.K, (uint32_t)k0};

  v16f acc[C::FM][C::FN];
  if (hi > lo)
    ring_mainloop<C>(smem, X, W, xs, ws, lo / BKS, (hi + BKS - 1) / BKS, lo, hi, acc);
  else
    zero_acc<C>(acc);
  // group bounds that are not multiples of 16 (any offsets are accepted, as
  // in the reference): the straddling chunks' in-group tokens
  if ((lo | hi) & 15) edge_chunks<C>(X, W, xs, ws, lo, hi, acc);

  if constexpr (PIECES) {
    store_partial<C>(acc, p.part + (int64_t)blockIdx.x * (C::BM * C::BN));
    return;
  }
  if constexpr (EPI == kEpiBf16) {
    store_tile_lds<C, true>(acc, smem, p.out + ((int64_t)g * p.N * p.K + n0 * p.K + k0) * 2, p.K, rows, cols);
  } else if constexpr (EPI == kEpiF16) {   // f16 of the bf16-rounded value
    store_tile_lds<C, false, true>(acc, smem, p.out + ((int64_t)g * p.N * p.K + n0 * p.K + k0) * 2, p.K, rows,
                                   cols);
  } else if constexpr (EPI == kEpiF16Any) {   // the same, rows off the 16-byte grid
    store_tile<C, true>(acc, p.out + ((int64_t)g * p.N * p.K + n0 * p.K + k0) * 2, p.K, rows, cols, MXGG_DTYPE_F16);
  } else {   // f32, or bf16 rows off the 16-byte grid (the type known to be one of the two)
    const int dt = p.out_dtype == MXGG_DTYPE_F32 ? MXGG_DTYPE_F32 : MXGG_DTYPE_BF16;
    const int esz = dt == MXGG_DTYPE_F32 ? 4 : 2;
    store_tile<C, true>(acc, p.out + ((int64_t)g * p.N * p.K + n0 * p.K + k0) * esz, p.K, rows, cols, dt);
  }
}

// Split tiles of a wgrad launch: one workgroup per item (v, c), as in
// fwd_reduce_kernel; items past the plan's split tiles exit.
template <class C>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(WgradParams p) {
  __shared__ __attribute__((aligned(16))) uint8_t blk[32 * C::WTN * 2];
  constexpr int CH = ReduceShape<C>::CH;
  const int v = blockIdx.x / CH, f = (blockIdx.x % CH) * 4 + wave_id();
  int lt, base, S;
  if (!wgrad_split_tile<C>(p, v, lt, base, S)) return;
  const int lane = threadIdx.x % kWave;
  const WgradTile tl = wgrad_tile<C>(p, lt);
  float acc[16];
  sum_pieces<C>(p.part + (int64_t)base * (C::BM * C::BN), S, f, lane, acc);
  const int esz = p.out_dtype == MXGG_DTYPE_F32 ? 4 : 2;
  store_item<C, true>(acc, f, lane, p.out + ((int64_t)tl.g * p.N * p.K + tl.n0 * p.K + tl.k0) * esz, p.K, tl.rows,
                      tl.cols, p.out_dtype, blk);
}

// ---------------------------------------------------------------------------
// routing table / tile order: test hooks that run the GEMMs' own device code
// ---------------------------------------------------------------------------

// The reference's routing buffer [hist E | start E | total | map grid_m_ub]
// (kernels/forward.py:320-354), built with the lookup the GEMMs run: with
// one column tile and bands of one m-block, route_tile's order is the
// reference's m-block order, so tile t is m-block t of the map.  One wave.
__global__ __launch_bounds__(64) void routing_kernel(const int32_t* offs, int E, int BM, int grid_m_ub,
                                                     int32_t* out) {
  for (int e = threadIdx.x; e < E; e += kWave) {
    int prev = e > 0 ? offs[e - 1] : 0;
    out[e] = offs[e] - prev;
    out[E + e] = prev;
  }
  WaveGroups wg{0, 0, 0, 0, 0};
  int total;
  if (E <= kWave) {
    wg = load_groups(offs, E, BM);
    total = wg.total;
  } else {
    total = route_total(offs, E, BM);
  }
  if (threadIdx.x == 0) out[2 * E] = total;
  for (int pid = 0; pid < grid_m_ub; ++pid) {
    int pn;
    const TileRoute r = E <= kWave ? route_tile(wg, E, BM, 1, 1, pid, pn) : route_tile(offs, E, BM, 1, 1, pid, pn);
    if (threadIdx.x == 0) out[2 * E + 1 + pid] = r.expert >= 0 ? (r.block << 16) | r.expert : -1;
  }
}

// The forward kernels' tile order: for every program id of the whole-tile
// grid, the tile fwd_tile gives it (the XCD swizzle, then the expert-aligned
// bands of route_tile), as 5 int32s (expert, row0, rows, n0, cols), or -1s
// past the tiles.  One wave per workgroup, programs strided over the grid.
template <class C>
__global__ __launch_bounds__(64) void schedule_kernel(FwdParams p, int programs, int32_t* out) {
  WaveGroups wg;
  const int tiles = fwd_groups<C>(p, wg) * p.grid_n;
  for (int pid = blockIdx.x; pid < programs; pid += gridDim.x) {
    FwdTile tl;
    const bool ok = pid < tiles && fwd_tile<C>(p, pid, tiles, wg, tl);
    if (threadIdx.x < 5) {
      int v = -1;
      if (ok) {
        const int64_t f[5] = {tl.expert, tl.row0, tl.rows, tl.n0, tl.cols};
        v = (int)f[threadIdx.x];
      }
      out[5 * (int64_t)pid + threadIdx.x] = v;
    }
  }
}

}  // namespace mxgg

// ===========================================================================
// C ABI
// ===========================================================================

using namespace mxgg;

// Row stride of a weight staged in row pairs (K bytes rounded up to 64).
static int64_t staged_ld(int64_t K) { return (K + 63) / 64 * 64; }

// Extra workspace for staging an e4m3 weight in row pairs, or 0 where the
// call would not gain from it.  Staging copies the weight once (2 E N K
// bytes of HBM traffic in the re-layout launch the call makes anyway); the
// GEMM then copies whole 128-byte lines of it.  Measured over the sweep
// shapes (MI355X, M = 16640, whole drop-in calls): E = 1 and 2 gain 2-10%
// at K >= 5120 and 2-3% at K = 2048 with N >= 5120 (nothing at N = K = 2048);
// E = 4 gains on some shapes and loses up to 3% on others: the copy's time
// over the GEMM's is about 400 E / M (5 TB/s against 2 PFLOP/s), so
// E <= M / 8192.  256 bytes of slack keep the staged lines 256-byte aligned.
static size_t fwd_staging_bytes(int E, int64_t M, int64_t N, int64_t K, int b_fmt) {
  if (b_fmt != MXGG_FMT_E4M3 || E <= 0 || N <= 0 || N % 2 || (int64_t)E * 8192 > M) return 0;
  if (K < 2048 || (K < 4096 && N < 4096)) return 0;
  if ((int64_t)E * (N / 2) > (1 << 22) || K >= (1 << 22)) return 0;   // launch grid, int offsets
  return (size_t)E * (size_t)N * (size_t)staged_ld(K) + 256;
}

// Forward calls of at most this many multiply-adds (1.2e11 flop) that stage
// nothing run on plain scales without a re-layout launch (run_grouped_mm).
constexpr int64_t kPlainMaxMacs = (int64_t)60000000000;

// The same for A (M, K), or 0: its copy's time over the GEMM's is about
// 400 / N, and staging it paid at N >= 8192 on every sweep shape (drop-in
// call, same box: -1 to -12% at E = 4 and 8, where the weight is not staged;
// -0.1 to -6% at E = 1 and 2 on top of the staged weight; with e2m1
// weights, BASELINE config 5 -2.7%), not reliably at N = 5120 (-6% to
// +1.4%).  A is e4m3 whatever the weight's format.  Not on calls of at most
// kPlainMaxMacs: their re-layout launch costs more than the row pairs save
// (E = 1, M = 2080, N = 8192, K = 2048: 57.3 us staged, 52.6 us on plain
// scales and row-major A).
static size_t fwd_staging_bytes_a(int64_t M, int64_t N, int64_t K, int b_fmt) {
  if ((b_fmt != MXGG_FMT_E4M3 && b_fmt != MXGG_FMT_E2M1) || M <= 0 || M % 2 || N < 8192 || K < 2048) return 0;
  if (M / 2 > (1 << 22) || K >= (1 << 22)) return 0;   // launch grid, int offsets
  if (M * N <= kPlainMaxMacs / K) return 0;
  return (size_t)M * (size_t)staged_ld(K) + 256;
}

namespace {

typedef Cfg<256, 256, 2, 2, MXGG_FMT_E4M3, 4> CfgF8_256;
typedef Cfg<128, 128, 2, 2, MXGG_FMT_E4M3, 4> CfgF8_128;
// e2m1 weights: stages of 24 KB in a 4-deep ring, like e4m3 (a 5-deep ring
// measured the same on BASELINE config 5, 650 vs 651 us, and spilled 8 bytes
// per lane in the LDS-staged epilogues)
typedef Cfg<256, 256, 2, 2, MXGG_FMT_E2M1, 4> CfgF4_256;
// The same tiles on plain to_mx scales (drop-in calls whose scale rows are
// 16-byte multiples): no scale re-layout launch; 16 KB scale slots of 8 steps
// (8 KB for 128 x 128 tiles).
typedef Cfg<256, 256, 2, 2, MXGG_FMT_E4M3, 4, true> CfgF8_256P;
typedef Cfg<128, 128, 2, 2, MXGG_FMT_E4M3, 4, true> CfgF8_128P;
typedef Cfg<256, 256, 2, 2, MXGG_FMT_E2M1, 4, true> CfgF4_256P;
// 256 x 256 e4m3 tiles with X in two-stage slots, for row-major X (XLine)
typedef XLine<Cfg<256, 256, 2, 2, MXGG_FMT_E4M3, 3>> CfgF8_256X;

// The scale-independent kernels of a configuration (the reduce): its
// step-major twin.
template <class C>
using StepCfg = Cfg<C::BM, C::BN, C::WGM, C::WGN, C::WFMT, C::XD ? 4 : C::NS>;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct FwdChoice {
  int bm, bn, group_m, xcd;
  bool split;   // the last round may be split along K (workspace permitting)
};

struct TunedFwd {
  int E, M, N, K, b_fmt, bm, bn, group_m, xcd, split;
};

#include "tuned_fwd.h"

// Tuned entry for (E, M, N, K, b_fmt): same E, N, K and format, M within a
// factor of two of the swept M; null when the sweep did not cover the shape.
const TunedFwd* find_tuned(int E, int64_t M, int64_t N, int64_t K, int b_fmt) {
  for (const TunedFwd* t = kTunedFwd; t->E; ++t)
    if (t->E == E && t->N == N && t->K == K && t->b_fmt == b_fmt && 2 * M >= t->M && M <= 2 * (int64_t)t->M)
      return t;
  return nullptr;
}

// A tuned entry when the sweep covered the shape.  Otherwise 256 x 256
// tiles, the 8-XCD swizzle and expert-aligned bands of at most 12 m-blocks
// (route_tile; 12 beat 8 and 16 on the sweep's jagged groups, and the
// 256 x 256 tile beats 128 x 128 even at N = K = 2048); 128 x 128 tiles for
// e4m3 problems too small to fill half the chip with 256 x 256 tiles, unless
// the 256 x 256 plan splits that lone round along K.
// Requests (nonzero bm, bn, gm, xcd) override field by field, and any request
// leaves the split to the workspace (a tuned "whole tiles only" applies to
// calls that request nothing).
template <class C>
int fwd_resident();

// A tuned entry applies whole on every operand layout, although the sweep
// timed the drop-in call's (operands staged by the library's rule): calls on
// different layouts give the same bits, and the tile order can change them --
// the tiles of a split last round are the last ones in that order.
FwdChoice pick_fwd(int E, int64_t M, int64_t N, int64_t K, int b_fmt, int bm, int bn, int gm, int xcd) {
  FwdChoice c{256, 256, 12, 8, true};
  const int64_t tiles256 = (cdiv(M, 256) + E - 1) * cdiv(N, 256);
  const TunedFwd* t = find_tuned(E, M, N, K, b_fmt);
  if (t) {
    c = FwdChoice{t->bm, t->bn, t->group_m, t->xcd, t->split != 0};
  } else if (b_fmt == MXGG_FMT_E4M3 && tiles256 < 128) {
    // Under half a chip of 256 x 256 tiles: 128 x 128 tiles (two per CU)
    // spread the work over 4x the workgroups, unless the 256 x 256 launch
    // splits its lone round along K (a long reduction; judged for the full
    // workspace that mxgg_grouped_mm_workspace_size recommends).  E=1, M=2080 (one
    // GPU's share of E=8 under 8-way expert parallelism), N=2048: K=5120
    // 77 -> 54 us; K=8192 splits (70 us, against 76 us as 128 x 128).
    const int par = fwd_resident<CfgF8_256>();
    const int slots = (int)(kSplitBytes / ((size_t)256 * 256 * 4));
    if (split_plan((int)tiles256, par > 0 ? par : 256, (int)cdiv(K, STEP), slots, 256).units == 0) {
      c.bm = 128;
      c.bn = 128;
    }
  }
  if (bm || bn || gm || xcd) c.split = true;
  if (bm) c.bm = bm;
  if (bn) c.bn = bn;
  if (gm) c.group_m = gm;
  if (xcd) c.xcd = xcd;
  return c;
}

// Workgroups of `kernel` (nt threads) resident on the current device at
// once: CUs x per-CU occupancy (LDS, registers).  Cached per device.
template <class KF>
int resident_workgroups(KF kernel, int nt, int (&cache)[64]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (dev >= 0 && dev < 64 && cache[dev]) return cache[dev];
  int cus = 0, per = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, nt, 0) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const int r = cus * (per > 0 ? per : 1);
  if (dev >= 0 && dev < 64) cache[dev] = r;
  return r;
}

template <class C>
int fwd_resident() {
  static int cache[64];
  return resident_workgroups(fwd_kernel<C, false>, C::NT, cache);
}

// Partial slots of BM x BN fp32 available in `bytes` (capped).
template <class C>
int split_slots(size_t bytes) {
  const size_t n = bytes / ((size_t)C::BM * C::BN * 4);
  return n > 4096 ? 4096 : (int)n;
}

// Forward launch: the whole tiles (grid: every possible tile; those at or
// past dp exit), then, when the workspace allows a split at all, the pieces
// (grid: the most pieces a plan can have) and the reduce of the split tiles.
// The plan itself depends on offs and is made on the device.
template <class C>
int launch_fwd(const FwdParams& p0, int grid_m_ub, int gm, int xcd, size_t part_bytes, hipStream_t st) {
  FwdParams p = p0;
  p.grid_n = (int)cdiv(p.N, C::BN);
  p.group_m = gm;
  p.xcd = xcd;
  p.par = fwd_resident<C>();
  p.slots = p.part ? split_slots<C>(part_bytes) : 0;
  const int nsteps = (int)cdiv(p.K, STEP);
  if (p.par <= 0 || p.slots < 2 || nsteps < kMinSplitTotal) p.slots = 0;
  // Rows of every group add up to M in the usual MoE call, with half a tile
  // of padding per group on average: when the plan for that many tiles does
  // not split, the piece and reduce launches are skipped (p.slots = 0 makes
  // the device plan agree).  A wrong guess costs time, never correctness.
  if (p.slots) {
    const int64_t est = (cdiv(p.M, C::BM) + (p.E - 1) / 2) * p.grid_n;
    if (est > INT32_MAX || split_plan((int)est, p.par, nsteps, p.slots, C::BM * C::BN * 4 / 1024).units == 0)
      p.slots = 0;
  }
  // A reduction too short to split: the last round may run as 128 x 128
  // quarter tiles (quad_dp).  The device decides from the real tile count;
  // the host, from the usual one, only skips the launch where it cannot help.
  p.quads = 0;
  constexpr bool kQuads = std::is_same<C, CfgF8_256>::value || std::is_same<C, CfgF8_256P>::value ||
                          std::is_same<C, CfgF8_256X>::value;
  typedef typename std::conditional<C::PS, CfgF8_128P, CfgF8_128>::type Q;
  if constexpr (kQuads) {
    if (nsteps < kMinSplitTotal && p.par > 0) {
      const int64_t est = (cdiv(p.M, C::BM) + (p.E - 1) / 2) * p.grid_n;
      if (est <= INT32_MAX && quad_dp((int)est, p.par) < est) p.quads = 1;
    }
  }
  const int64_t tiles_ub = (int64_t)grid_m_ub * p.grid_n;
  if (tiles_ub <= 0) return MXGG_OK;
  if (tiles_ub > INT32_MAX) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: grid too large");
  // The device's tile count is m * grid_n for some m <= grid_m_ub (each
  // group adds whole m-blocks of grid_n tiles).  When every such count is
  // below one round and its plan splits, no tile runs whole: the whole-tile
  // launch would only route and exit (4.5 us on the expert-parallel shard's
  // N = 2048, K = 8192 call), so it is left out.
  bool whole = true;
  if (p.slots && tiles_ub < p.par) {
    whole = false;
    for (int m = 1; m <= grid_m_ub && !whole; ++m)
      if (split_plan(m * p.grid_n, p.par, nsteps, p.slots, C::BM * C::BN * 4 / 1024).units == 0) whole = true;
  }
  const int epi = pick_epi(p.out_dtype, p.ldo, p.out);
  if (whole) switch (epi) {
#define MXGG_WHOLE(E) \
  case E: hipLaunchKernelGGL((fwd_kernel<C, false, E>), dim3((unsigned)tiles_ub), dim3(C::NT), 0, st, p); break
    MXGG_WHOLE(kEpiBf16);
    MXGG_WHOLE(kEpiF16);
    MXGG_WHOLE(kEpiF32);
    MXGG_WHOLE(kEpiBf16Any);
    MXGG_WHOLE(kEpiF16Any);
#undef MXGG_WHOLE
  }
  if (int rc = launch_status("grouped_mm")) return rc;
  if constexpr (kQuads) {
    if (p.quads) {   // 4 * (T % P) <= P quarters
      switch (epi) {
#define MXGG_QUAD(E)                                                                                         \
  case E:                                                                                                   \
    hipLaunchKernelGGL((fwd_quad_kernel<C, Q, E>), dim3((unsigned)p.par), dim3(Q::NT), 0, st, p); \
    break
        MXGG_QUAD(kEpiBf16);
        MXGG_QUAD(kEpiF16);
        MXGG_QUAD(kEpiF32);
        MXGG_QUAD(kEpiBf16Any);
        MXGG_QUAD(kEpiF16Any);
#undef MXGG_QUAD
      }
      if (int rc = launch_status("grouped_mm")) return rc;
    }
  }
  if (!p.slots) return MXGG_OK;
  const int pieces = p.slots;   // units = rem * S <= slots
  hipLaunchKernelGGL((fwd_kernel<C, true>), dim3((unsigned)pieces), dim3(C::NT), 0, st, p);
  if (int rc = launch_status("grouped_mm")) return rc;
  // a split needs rem <= par / 2 tiles of ReduceShape::CH items each; the
  // grid strides over them.  One workgroup per item of the split the host
  // expects (at least 128, which costs little when the device plan differs):
  // a 72-tile split (1152 items) took 21 us on 128 workgroups.
  const int64_t items = (int64_t)(p.par / 2) * ReduceShape<C>::CH;
  const int64_t est = (cdiv(p.M, C::BM) + (p.E - 1) / 2) * p.grid_n;
  const Split esp = split_plan((int)(est < INT32_MAX ? est : INT32_MAX), p.par, nsteps, p.slots,
                               C::BM * C::BN * 4 / 1024);
  int64_t rgrid = esp.S > 0 ? (int64_t)(esp.units / esp.S) * ReduceShape<C>::CH : 0;
  if (rgrid < 128) rgrid = 128;
  if (rgrid > items) rgrid = items;
  if (rgrid <= 0) return MXGG_OK;
  hipLaunchKernelGGL((fwd_reduce_kernel<StepCfg<C>>), dim3((unsigned)rgrid), dim3(256), 0, st, p);
  return launch_status("grouped_mm");
}

ScaleJob scale_job(const uint8_t* src, int64_t ld_r, int64_t ld_b, uint32_t* dst, int64_t rows,
                   int batches, int64_t nblk, int64_t steps) {
  ScaleJob j{src, ld_r, ld_b, dst, (int)rows, batches, (int)nblk, (int)steps,
             (int)cdiv(rows, 64), (int)cdiv(steps, 16)};
  return j;
}

// Re-lay two operands' scales into the workspace, and, given pair jobs,
// one or two operands' data into row pairs (one launch).
int launch_relayout(const ScaleJob& a, const ScaleJob& b, hipStream_t st, const char* what,
                    const PairJob* d = nullptr, const PairJob* d2 = nullptr) {
  ScaleJobs js;
  js.j[0] = a;
  js.j[1] = b;
  js.tiles0 = a.batches * a.tiles_r * a.tiles_t;
  const int64_t t01 = (int64_t)js.tiles0 + (int64_t)b.batches * b.tiles_r * b.tiles_t;
  if (t01 > INT32_MAX) return fail(MXGG_ERR_UNSUPPORTED, "%s: scale re-layout grid too large", what);
  js.tiles01 = (int)t01;
  js.d = d ? *d : PairJob{};
  js.tiles_d = d ? d->batches * d->pairs : 0;
  js.d2 = d2 ? *d2 : PairJob{};
  const int64_t grid = t01 + js.tiles_d + (d2 ? (int64_t)d2->batches * d2->pairs : 0);
  if (grid <= 0) return MXGG_OK;
  if (grid > (int64_t)(UINT32_MAX / 256)) return fail(MXGG_ERR_UNSUPPORTED, "%s: re-layout grid too large", what);
  if (grid > INT32_MAX) return fail(MXGG_ERR_UNSUPPORTED, "%s: scale re-layout grid too large", what);
  hipLaunchKernelGGL(scale_relayout_kernel, dim3((unsigned)grid), dim3(256), 0, st, js);
  return launch_status(what);
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
  if (M < 0 || N < 0 || M > INT32_MAX || N > INT32_MAX)
    return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: M, N out of range");
  if (group_m <= 0 || xcd_swizzle <= 0)
    return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: group_m and xcd_swizzle must be positive");
  if (!((block_m == 256 && block_n == 256) || (block_m == 128 && block_n == 128)))
    return fail(MXGG_ERR_UNSUPPORTED, "tile_schedule: tile %dx%d not built", block_m, block_n);
  const int64_t programs = mxgg_schedule_programs(E, M, N, block_m, block_n);
  if (programs > INT32_MAX / 5) return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: too many programs");
  if (!offs || !out) return fail(MXGG_ERR_INVALID_ARG, "tile_schedule: null pointer");
  if (int rc = require_device()) return rc;
  if (programs == 0) return MXGG_OK;
  FwdParams p{};
  p.offs = offs;
  p.E = E;
  p.M = M;
  p.N = N;
  p.grid_n = (int)cdiv(N, block_n);
  p.group_m = group_m;
  p.xcd = xcd_swizzle;
  const unsigned grid = (unsigned)(programs < 1024 ? programs : 1024);
  if (block_m == 256)
    hipLaunchKernelGGL(schedule_kernel<CfgF8_256>, dim3(grid), dim3(64), 0, (hipStream_t)stream, p, (int)programs,
                       out);
  else
    hipLaunchKernelGGL(schedule_kernel<CfgF8_128>, dim3(grid), dim3(64), 0, (hipStream_t)stream, p, (int)programs,
                       out);
  return launch_status("tile_schedule");
}

static bool aligned16(const void* p) { return ((uintptr_t)p % 16) == 0; }

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Re-laid scales of a forward call: A [T][M], then B [E][T][N] dwords.
static size_t fwd_scale_bytes(int E, int64_t M, int64_t N, int64_t K) {
  return (size_t)4 * (size_t)cdiv(K, STEP) * ((size_t)M + (size_t)E * (size_t)N);
}

// Partial-tile area worth reserving: up to kSplitBytes, no more than `tiles`
// tiles of `tile_bytes` cut into the most pieces a reduction of `nsteps`
// steps allows.
static size_t split_area(int64_t tiles, size_t tile_bytes, int64_t nsteps) {
  if (nsteps < kMinSplitTotal || tiles <= 0) return 0;
  int64_t smax = nsteps / kMinSplitSteps;
  if (smax > kMaxSplit) smax = kMaxSplit;
  const double want = (double)tiles * (double)smax * (double)tile_bytes;
  return want < (double)kSplitBytes ? (size_t)want : kSplitBytes;
}

// Extra workspace for staging both wgrad operands (go_t (N, M), ia_t (K, M))
// in row pairs, or 0 where that would not pay.  The copy moves 2 (N + K) M
// bytes in the scale re-layout launch; the GEMM then copies whole lines of
// both operands, where on row-major data the XLine kernel copies whole lines
// of go_t only (kernel-only, row pairs are 13% faster over the sweep).  The
// copy's time over the GEMM's is about 2000 (N + K) / (N K), so it pays only
// at N = K = 8192; with 8 or more groups, whose token ranges are short, also
// at N + K >= 10240.  Measured on the whole drop-in call against staging every
// shape (MI355X, M = 16640, 36 sweep shapes, same bits on all): -2.1%
// geomean; without any staging -1.6% (the unstaged calls up to 10% faster,
// E = 8 at N + K >= 10240 and N = K = 8192 1-4% slower).
static size_t wgrad_staging_bytes(int E, int64_t M, int64_t N, int64_t K) {
  if (E <= 0 || M <= 0 || M % 32 || N <= 0 || K <= 0 || N % 2 || K % 2) return 0;
  if (!((N >= 8192 && K >= 8192) || (E >= 8 && N + K >= 10240))) return 0;
  if (M >= (1 << 22) || N / 2 + K / 2 > (1 << 22)) return 0;   // int offsets, launch grid
  return (size_t)(N + K) * (size_t)staged_ld(M) + 512;
}

extern "C" size_t mxgg_wgrad_staging_size(int E, int64_t M, int64_t N, int64_t K) {
  return wgrad_staging_bytes(E, M, N, K);
}

extern "C" size_t mxgg_grouped_mm_staging_size(int E, int64_t M, int64_t N, int64_t K, int b_fmt) {
  if (M < 0 || K < 0 || K % 32 || E <= 0) return 0;
  return fwd_staging_bytes(E, M, N, K, b_fmt) + fwd_staging_bytes_a(M, N, K, b_fmt);
}

// Partial-tile room of a forward call: the most a split plan of the call can
// use (256 x 256 or 128 x 128 tiles, whichever needs more).  Calls given more
// use no more, so every call with at least this room makes the same plan.
static size_t fwd_part_cap(int E, int64_t M, int64_t N, int64_t K) {
  if (E <= 0 || M <= 0 || N <= 0 || K <= 0) return 0;
  const int64_t nsteps = cdiv(K, STEP);
  const size_t a = split_area((cdiv(M, 256) + E - 1) * cdiv(N, 256), (size_t)256 * 256 * 4, nsteps);
  const size_t b = split_area((cdiv(M, 128) + E - 1) * cdiv(N, 128), (size_t)128 * 128 * 4, nsteps);
  return a > b ? a : b;
}

extern "C" size_t mxgg_grouped_mm_workspace_size(int E, int64_t M, int64_t N, int64_t K) {
  if (E <= 0 || M < 0 || N < 0 || K < 0) return 0;
  const size_t sc = fwd_scale_bytes(E, M, N, K);
  if (sc == 0 || M == 0 || N == 0) return sc;
  const size_t part = fwd_part_cap(E, M, N, K);
  return part ? align256(sc) + part : sc;
}

// Where the parts of a caller's workspace go (plain-scale entry points): the
// re-laid scales (`need` bytes) first; then, 256-byte aligned, the partial
// tiles, given at most `cap` bytes; then, from the bytes past those, the
// staged operands (`stage` bytes, carved from the end).  A workspace of the
// recommended size therefore stages nothing, and a larger one stages without
// taking room from the partial tiles: the split plan, and the bits, are those
// of the unstaged call.
struct WsLayout {
  size_t part_off;    // first byte of the partial area
  size_t part;        // its bytes (0: no tile is split)
  size_t extra;       // bytes past the scales and the partial area
};

static WsLayout ws_layout(size_t ws_bytes, size_t need, size_t cap) {
  WsLayout w{align256(need), 0, 0};
  const size_t avail = ws_bytes > w.part_off ? ws_bytes - w.part_off : 0;
  w.part = avail < cap ? avail : cap;
  const size_t used = w.part ? w.part_off + w.part : need;
  w.extra = ws_bytes > used ? ws_bytes - used : 0;
  return w;
}

// Bytes a row of `len` bytes takes in an operand stored in pieces of `piece`
// bytes (64 for row pairs, 32 for row quads, 1 for rows).
static int64_t operand_row_bytes(int64_t len, int64_t piece) { return (len + piece - 1) / piece * piece; }

// Argument checks of a forward call shared by the entry points; MXGG_OK
// when the call may go ahead (check *empty: nothing to compute).
// plain: A_s / B_s are plain scales with these strides (else step-major,
// strides unused).  layout: MXGG_A_PAIRS / MXGG_B_PAIRS flags.
static int check_grouped_mm(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas, const uint8_t* B,
                            int b_fmt, int64_t ldb_n, int64_t ldb_e, const uint8_t* B_s, int64_t ldbs_n,
                            int64_t ldbs_e, const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                            const void* out, int out_dtype, int64_t ldo, bool plain, int layout, bool* empty) {
  *empty = false;
  if (b_fmt != MXGG_FMT_E4M3 && b_fmt != MXGG_FMT_E2M1)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: weight format %d not E4M3/E2M1", b_fmt);
  if (layout & ~(MXGG_A_PAIRS | MXGG_B_PAIRS | MXGG_B_QUADS) || (layout & MXGG_B_PAIRS && layout & MXGG_B_QUADS))
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: unknown operand layout flags %d", layout);
  const bool ap = layout & MXGG_A_PAIRS, bp = layout & MXGG_B_PAIRS, bq = layout & MXGG_B_QUADS;
  if (bp && b_fmt != MXGG_FMT_E4M3)
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: row pairs are built for e4m3 weights only (e2m1: row quads)");
  if (bq && b_fmt != MXGG_FMT_E2M1)
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: row quads are built for packed e2m1 weights only (e4m3: row pairs)");
  if ((ap && M % 2) || (bp && N % 2) || (bq && N % 4))
    return fail(MXGG_ERR_INVALID_ARG,
                "grouped_mm: an operand in row pairs / quads needs a row count divisible by 2 / 4 (M=%lld, N=%lld)",
                (long long)M, (long long)N);
  if (out_dtype != MXGG_DTYPE_BF16 && out_dtype != MXGG_DTYPE_F16 && out_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: out_dtype %d not BF16/F16/F32", out_dtype);
  if (E <= 0 || E > 65535) return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: E=%d out of range", E);
  if (M < 0 || N < 0 || K < 0) return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: negative shape");
  if (K % 32) return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: K=%lld must be a multiple of 32", (long long)K);
  const int64_t kb = b_fmt == MXGG_FMT_E2M1 ? K / 2 : K;
  if (lda < operand_row_bytes(K, ap ? 64 : 1) || ldb_n < operand_row_bytes(kb, bp ? 64 : (bq ? 32 : 1)) || ldo < N ||
      (plain && (ldas < K / 32 || ldbs_n < K / 32)))
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: a row stride is smaller than its row");
  if (E > 1 && (ldb_e < N * ldb_n || (plain && ldbs_e < N * ldbs_n)))
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: expert stride smaller than one expert");
  if (lda % 16 || ldb_n % 16 || !aligned16(A) || !aligned16(B))
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: A/B rows must be 16-byte aligned");
  if (lda >= (1 << 23) || ldb_n >= (1 << 23))
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: row strides must be below 2**23 bytes");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: dimension above 2**31");
  if (M == 0 || N == 0) {
    *empty = true;
    return MXGG_OK;
  }
  if (!A || !A_s || !B || !B_s || !offs || !out)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm: null pointer");
  if (fwd_scale_bytes(E, M, N, K) >= ((size_t)1 << 31))
    return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: problem too large");
  return MXGG_OK;
}

// Plain to_mx scales the GEMMs can read directly (plain-scale kernels): rows
// of 16-byte multiples, 16-byte aligned buffers, byte ranges below 2**31.
static bool plain_scales_ok(const uint8_t* A_s, int64_t ldas, const uint8_t* B_s, int64_t ldbs_n, int64_t ldbs_e,
                            int E, int64_t M, int64_t N) {
  if (ldas % 16 || ldbs_n % 16 || (E > 1 && ldbs_e % 16) || !aligned16(A_s) || !aligned16(B_s)) return false;
  const int64_t bexp = E > 1 ? ldbs_e : N * ldbs_n;
  return M * ldas < ((int64_t)1 << 31) && bexp < ((int64_t)1 << 31) && (int64_t)(E - 1) * bexp < ((int64_t)1 << 40);
}

// The GEMM launches of a checked forward call on step-major scales (as: A
// [T][M], bs: B [E][T][N] dwords), or, with `plain`, on plain to_mx scales
// (as: A (M, K/32) with row stride ldas, bs: B (E, N, K/32) with strides
// ldbs_n, ldbs_e; plain_scales_ok holds); part / part_bytes: room for the fp32
// partial tiles of a split last round (none: no tile is split).
static int launch_grouped_mm(const uint8_t* A, int64_t lda, const uint8_t* as, const uint8_t* B, int b_fmt,
                             int64_t ldb_n, int64_t ldb_e, const uint8_t* bs, const int32_t* offs, int E, int64_t M,
                             int64_t N, int64_t K, void* out, int out_dtype, int64_t ldo, int block_m, int block_n,
                             int group_m, int xcd, int layout, void* part_area, size_t part_bytes, hipStream_t st,
                             bool plain = false, int64_t ldas = 0, int64_t ldbs_n = 0, int64_t ldbs_e = 0) {
  FwdChoice c = pick_fwd(E, M, N, K, b_fmt, block_m, block_n, group_m, xcd);
  const bool built = b_fmt == MXGG_FMT_E2M1 ? (c.bm == 256 && c.bn == 256)
                                           : ((c.bm == 256 && c.bn == 256) || (c.bm == 128 && c.bn == 128));
  if (!built) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm: tile %dx%d not built", c.bm, c.bn);
  const int64_t T = cdiv(K, STEP);
  float* part = c.split && part_area && part_bytes ? (float*)part_area : nullptr;
  FwdParams p{A, lda, B, ldb_n, ldb_e, as, (uint32_t)(4 * T * M), bs, (uint32_t)(4 * T * N), offs, E, M, N, K,
              (uint8_t*)out, out_dtype, ldo, 0, 0, 0, part, 0, 0, 0,
              (layout & MXGG_A_PAIRS) ? 1 : 0, (layout & MXGG_B_PAIRS) ? 1 : ((layout & MXGG_B_QUADS) ? 2 : 0)};
  // no more room than the split plans of this shape can use (ws_layout)
  const size_t cap = fwd_part_cap(E, M, N, K);
  const size_t pb = part ? (part_bytes < cap ? part_bytes : cap) : 0;
  if (!pb) part = nullptr;
  p.part = part;
  const int gm256 = (int)(cdiv(M, 256) + E - 1), gm128 = (int)(cdiv(M, 128) + E - 1);
  if (plain) {
    p.as_bytes = (uint32_t)(M * ldas);
    p.bs_expert = (uint32_t)(E > 1 ? ldbs_e : N * ldbs_n);
    p.as_ld = (uint32_t)ldas;
    p.bs_ld = (uint32_t)ldbs_n;
    if (b_fmt == MXGG_FMT_E2M1) return launch_fwd<CfgF4_256P>(p, gm256, c.group_m, c.xcd, pb, st);
    if (c.bm == 256) return launch_fwd<CfgF8_256P>(p, gm256, c.group_m, c.xcd, pb, st);
    return launch_fwd<CfgF8_128P>(p, gm128, c.group_m, c.xcd, pb, st);
  }
  if (b_fmt == MXGG_FMT_E2M1) return launch_fwd<CfgF4_256>(p, gm256, c.group_m, c.xcd, pb, st);
  if (c.bm == 256 && p.a_pl == 0) return launch_fwd<CfgF8_256X>(p, gm256, c.group_m, c.xcd, pb, st);
  if (c.bm == 256) return launch_fwd<CfgF8_256>(p, gm256, c.group_m, c.xcd, pb, st);
  return launch_fwd<CfgF8_128>(p, gm128, c.group_m, c.xcd, pb, st);
}

// A checked forward call on plain scales: the GEMM launches, on the plain
// scales where plain_scales_ok holds, else after re-laying them step-major
// into the workspace (the partial tiles follow the room of those scales in
// either case, so both ways make the same split plan and the same bits).
static int run_grouped_mm(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas, const uint8_t* B,
                          int b_fmt, int64_t ldb_n, int64_t ldb_e, const uint8_t* B_s, int64_t ldbs_n,
                          int64_t ldbs_e, const int32_t* offs, int E, int64_t M, int64_t N, int64_t K, void* out,
                          int out_dtype, int64_t ldo, int block_m, int block_n, int group_m, int xcd,
                          void* workspace, size_t ws_bytes, void* stream) {
  const size_t need = fwd_scale_bytes(E, M, N, K);
  hipStream_t st = (hipStream_t)stream;
  const int64_t T = cdiv(K, STEP);
  uint32_t* wsd = (uint32_t*)workspace;
  const WsLayout wl = ws_layout(ws_bytes, need, fwd_part_cap(E, M, N, K));
  // The weight, then A, in row pairs, staged at the end of the workspace
  // (the weight last) from the bytes past the partial area (ws_layout).
  const size_t stage_b = fwd_staging_bytes(E, M, N, K, b_fmt), stage_a = fwd_staging_bytes_a(M, N, K, b_fmt);
  const int ldp = (int)staged_ld(K);
  // (each staging size holds 256 bytes of slack for aligning its start)
  uint8_t* const end = (uint8_t*)workspace + ws_bytes;
  PairJob pb{}, pa{};
  const bool staged_b = T > 0 && stage_b && wl.extra >= stage_b;
  if (staged_b) pb = PairJob{B, ldb_n, ldb_e, (uint8_t*)align256((size_t)(end - stage_b)), ldp, (int)(N / 2), E, (int)K};
  const size_t used_b = staged_b ? stage_b : 0;
  const bool staged_a = T > 0 && stage_a && wl.extra >= used_b + stage_a;
  if (staged_a)
    pa = PairJob{A, lda, 0, (uint8_t*)align256((size_t)(end - used_b - stage_a)), ldp, (int)(M / 2), 1, (int)K};
  // The plain-scale kernels save the scale re-layout launch (4.4 us at the
  // least, a quarter of the smallest expert-parallel shard call) but copy
  // their scales in 32-byte row pieces, four times the copy requests of the
  // step-major dwords, which slows the main loop by about 3%.  Measured on
  // MI355X (drop-in forward, same bits either way): E = 1, M = 2080 calls of
  // 1.7e10 .. 1.1e11 flop -13 to -1.5%, 1.7e11 +0.6 to +2.6%, and the
  // 36-shape sweep (1.4e11 flop and up) +2.7% geomean.  So they run on calls
  // that stage nothing (staging launches the re-layout kernel anyway) of at
  // most kPlainMaxMacs multiply-adds.
  const bool plain = !staged_a && !staged_b && M * N <= kPlainMaxMacs / (K > 0 ? K : 1) &&
                     plain_scales_ok(A_s, ldas, B_s, ldbs_n, ldbs_e, E, M, N);
  if (T > 0 && !plain) {
    if (int rc = launch_relayout(scale_job(A_s, ldas, 0, wsd, M, 1, K / 32, T),
                                 scale_job(B_s, ldbs_n, ldbs_e, wsd + T * M, N, E, K / 32, T), st, "grouped_mm",
                                 staged_b ? &pb : nullptr, staged_a ? &pa : nullptr))
      return rc;
  }
  void* part = wl.part ? (void*)((uint8_t*)workspace + wl.part_off) : nullptr;
  return launch_grouped_mm(staged_a ? pa.dst : A, staged_a ? (int64_t)ldp : lda,
                           plain ? A_s : (const uint8_t*)wsd, staged_b ? pb.dst : B, b_fmt,
                           staged_b ? (int64_t)ldp : ldb_n, staged_b ? N * ldp : ldb_e,
                           plain ? B_s : (const uint8_t*)(wsd + T * M), offs, E, M, N, K, out, out_dtype, ldo,
                           block_m, block_n, group_m, xcd, (staged_b ? MXGG_B_PAIRS : 0) | (staged_a ? MXGG_A_PAIRS : 0),
                           part, wl.part, st, plain, ldas, ldbs_n, ldbs_e);
}

extern "C" int mxgg_grouped_mm(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas,
                               const uint8_t* B, int b_fmt, int64_t ldb_n, int64_t ldb_e,
                               const uint8_t* B_s, int64_t ldbs_n, int64_t ldbs_e,
                               const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                               void* out, int out_dtype, int64_t ldo, int block_m, int block_n,
                               int group_m, int xcd, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  bool empty;
  if (int rc = check_grouped_mm(A, lda, A_s, ldas, B, b_fmt, ldb_n, ldb_e, B_s, ldbs_n, ldbs_e, offs, E, M, N, K,
                                out, out_dtype, ldo, true, 0, &empty))
    return rc;
  if (empty) return MXGG_OK;
  const size_t need = fwd_scale_bytes(E, M, N, K);
  if (need && (!workspace || ws_bytes < need))
    return fail(MXGG_ERR_WORKSPACE, "grouped_mm: workspace of at least %zu bytes needed, %zu given", need,
                workspace ? ws_bytes : (size_t)0);
  if (int rc = require_device()) return rc;
  return run_grouped_mm(A, lda, A_s, ldas, B, b_fmt, ldb_n, ldb_e, B_s, ldbs_n, ldbs_e, offs, E, M, N, K, out,
                        out_dtype, ldo, block_m, block_n, group_m, xcd, workspace, ws_bytes, stream);
}

extern "C" int mxgg_grouped_mm_steps(const uint8_t* A, int64_t lda, const uint32_t* A_ss, const uint8_t* B,
                                     int b_fmt, int64_t ldb_n, int64_t ldb_e, const uint32_t* B_ss,
                                     const int32_t* offs, int E, int64_t M, int64_t N, int64_t K, void* out,
                                     int out_dtype, int64_t ldo, int block_m, int block_n, int group_m, int xcd,
                                     int layout, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  bool empty;
  if (int rc = check_grouped_mm(A, lda, (const uint8_t*)A_ss, 0, B, b_fmt, ldb_n, ldb_e, (const uint8_t*)B_ss, 0, 0,
                                offs, E, M, N, K, out, out_dtype, ldo, false, layout, &empty))
    return rc;
  if (empty) return MXGG_OK;
  if (((uintptr_t)A_ss | (uintptr_t)B_ss) & 3)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm_steps: step-major scales must be 4-byte aligned");
  if (int rc = require_device()) return rc;
  return launch_grouped_mm(A, lda, (const uint8_t*)A_ss, B, b_fmt, ldb_n, ldb_e, (const uint8_t*)B_ss, offs, E, M,
                           N, K, out, out_dtype, ldo, block_m, block_n, group_m, xcd, layout, workspace,
                           workspace ? ws_bytes : 0, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// allocation-free forward entry point: the workspace is a device array of
// this library (one per GPU) instead of caller memory
// ---------------------------------------------------------------------------

// MXGG_NOALLOC_SCRATCH_BYTES per device, held from the library's load to the
// end of the process: the re-laid scales of a call (4 * cdiv(K, 128) *
// (M + E*N) bytes; 21 MB for the largest sweep shape), after them the fp32
// partial tiles of a split last round, and, at the end, a weight staged in
// row pairs when that fits as well (as for a caller's workspace of this
// size).  Nothing in it needs clearing: every call writes the scales and the
// staged weight before reading them, and a split call writes every partial
// tile before the reduce reads it.
static __device__ __align__(256) uint8_t scratch[MXGG_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64];   // device address of `scratch` per device; null until looked up
}  // namespace

// This device's copy of `scratch` (the host-side name is not a device
// address): looked up once per device, with that device current.
static int scratch_for_device(void** ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MXGG_ERR_NO_DEVICE, "grouped_mm_noalloc: no HIP device: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm_noalloc: device %d above 63", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(e != hipSuccess ? (int)e : MXGG_ERR_UNSUPPORTED, "grouped_mm_noalloc: hipGetSymbolAddress: %s",
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return MXGG_OK;
}

extern "C" int mxgg_grouped_mm_noalloc(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas,
                                       const uint8_t* B, int b_fmt, int64_t ldb_n, int64_t ldb_e,
                                       const uint8_t* B_s, int64_t ldbs_n, int64_t ldbs_e,
                                       const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                                       void* out, int out_dtype, int64_t ldo, int block_m, int block_n,
                                       int group_m, int xcd, void* stream) {
  clear_error();
  bool empty;
  if (int rc = check_grouped_mm(A, lda, A_s, ldas, B, b_fmt, ldb_n, ldb_e, B_s, ldbs_n, ldbs_e, offs, E, M, N, K,
                                out, out_dtype, ldo, true, 0, &empty))
    return rc;
  if (empty) return MXGG_OK;
  const size_t need = fwd_scale_bytes(E, M, N, K);
  if (need > (size_t)MXGG_NOALLOC_SCRATCH_BYTES)
    return fail(MXGG_ERR_WORKSPACE,
                "grouped_mm_noalloc: the re-laid scales need %zu bytes, more than the %zu-byte scratch "
                "(4 * cdiv(K, 128) * (M + E*N) must stay within it)",
                need, (size_t)MXGG_NOALLOC_SCRATCH_BYTES);
  if (int rc = require_device()) return rc;
  void* ws = nullptr;
  if (int rc = scratch_for_device(&ws)) return rc;
  return run_grouped_mm(A, lda, A_s, ldas, B, b_fmt, ldb_n, ldb_e, B_s, ldbs_n, ldbs_e, offs, E, M, N, K, out,
                        out_dtype, ldo, block_m, block_n, group_m, xcd, ws, (size_t)MXGG_NOALLOC_SCRATCH_BYTES,
                        stream);
}

extern "C" int mxgg_grouped_mm_config(int E, int64_t M, int64_t N, int64_t K, int b_fmt, int* block_m,
                                      int* block_n, int* group_m, int* xcd_swizzle) {
  clear_error();
  if (!block_m || !block_n || !group_m || !xcd_swizzle)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm_config: null output pointer");
  if (b_fmt != MXGG_FMT_E4M3 && b_fmt != MXGG_FMT_E2M1)
    return fail(MXGG_ERR_INVALID_ARG, "grouped_mm_config: weight format %d not E4M3/E2M1", b_fmt);
  FwdChoice c = pick_fwd(E, M, N, K, b_fmt, *block_m, *block_n, *group_m,
                         *xcd_swizzle);
  *block_m = c.bm;
  *block_n = c.bn;
  *group_m = c.group_m;
  *xcd_swizzle = c.xcd;
  const bool built = b_fmt == MXGG_FMT_E2M1 ? (c.bm == 256 && c.bn == 256)
                                           : ((c.bm == 256 && c.bn == 256) || (c.bm == 128 && c.bn == 128));
  if (!built) return fail(MXGG_ERR_UNSUPPORTED, "grouped_mm_config: tile %dx%d not built", c.bm, c.bn);
  return MXGG_OK;
}

// Re-laid scales of a wgrad call: GO [T][N], then IA [T][K] dwords.
static size_t wgrad_scale_bytes(int64_t M, int64_t N, int64_t K) {
  return (size_t)4 * (size_t)cdiv(M, STEP) * ((size_t)N + (size_t)K);
}

// Reduction steps of an average group (what the split plan is sized for).
static int64_t wgrad_group_steps(int E, int64_t M) {
  const int64_t n = cdiv(M, (int64_t)E * STEP);
  return n > 0 ? n : 1;
}

// Partial-tile room of a wgrad call: the most its split plan can use.  With
// several groups the kernels plan a lone under-filled round from the longest
// group, which may hold all M tokens: room for that plan.
static size_t wgrad_part_cap(int E, int64_t M, int64_t N, int64_t K) {
  if (E <= 0 || M <= 0 || N <= 0 || K <= 0) return 0;
  return split_area((int64_t)E * cdiv(N, 256) * cdiv(K, 256), (size_t)256 * 256 * 4,
                    E > 1 ? cdiv(M, STEP) : wgrad_group_steps(E, M));
}

extern "C" size_t mxgg_wgrad_workspace_size(int E, int64_t M, int64_t N, int64_t K) {
  if (E <= 0 || M < 0 || N < 0 || K < 0) return 0;
  const size_t sc = wgrad_scale_bytes(M, N, K);
  if (sc == 0 || N == 0 || K == 0) return sc;
  const size_t part = wgrad_part_cap(E, M, N, K);
  return part ? align256(sc) + part : sc;
}

// Argument checks of a wgrad call (plain: go_s / ia_s are plain scales with
// these strides); *empty: nothing to compute.
static int check_wgrad(const uint8_t* go_t, int64_t ld_go, const uint8_t* go_s, int64_t ld_gos, const uint8_t* ia_t,
                       int64_t ld_ia, const uint8_t* ia_s, int64_t ld_ias, const int32_t* offs, int E, int64_t M,
                       int64_t N, int64_t K, const void* out, int out_dtype, bool plain, int layout, bool* empty) {
  *empty = false;
  if (out_dtype != MXGG_DTYPE_BF16 && out_dtype != MXGG_DTYPE_F16 && out_dtype != MXGG_DTYPE_F32)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: out_dtype %d not BF16/F16/F32", out_dtype);
  if (E <= 0 || E > 65535) return fail(MXGG_ERR_INVALID_ARG, "wgrad: E=%d out of range", E);
  if (M < 0 || N < 0 || K < 0) return fail(MXGG_ERR_INVALID_ARG, "wgrad: negative shape");
  if (M % 32) return fail(MXGG_ERR_INVALID_ARG, "wgrad: M=%lld must be a multiple of 32", (long long)M);
  if (layout & ~(MXGG_A_PAIRS | MXGG_B_PAIRS))
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: unknown operand layout flags %d", layout);
  const bool gp = layout & MXGG_A_PAIRS, ip = layout & MXGG_B_PAIRS;
  if ((gp && N % 2) || (ip && K % 2))
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: an operand in row pairs needs an even row count (N=%lld, K=%lld)",
                (long long)N, (long long)K);
  if (ld_go < operand_row_bytes(M, gp ? 64 : 1) || ld_ia < operand_row_bytes(M, ip ? 64 : 1) ||
      (plain && (ld_gos < M / 32 || ld_ias < M / 32)))
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: a row stride is smaller than its row");
  if (ld_go % 16 || ld_ia % 16 || !aligned16(go_t) || !aligned16(ia_t))
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: operand rows must be 16-byte aligned");
  if (ld_go >= (1 << 23) || ld_ia >= (1 << 23))
    return fail(MXGG_ERR_UNSUPPORTED, "wgrad: row strides must be below 2**23 bytes");
  if (M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXGG_ERR_UNSUPPORTED, "wgrad: dimension above 2**31");
  if (N == 0 || K == 0) {
    *empty = true;
    return MXGG_OK;
  }
  if (!go_t || !go_s || !ia_t || !ia_s || !offs || !out)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad: null pointer");
  if (wgrad_scale_bytes(M, N, K) >= ((size_t)1 << 31)) return fail(MXGG_ERR_UNSUPPORTED, "wgrad: problem too large");
  return MXGG_OK;
}

// A wgrad launch whose 256 x 256 tiles would fill at most half the chip and
// whose plan cuts none of them (a reduction too short to split, e.g. one GPU's
// expert-parallel share, 2080 tokens, at N = K = 2048: 64 tiles on 256 CUs),
// or whose 128 x 128 tiles fill at least one round even where a split is
// planned (E = 2, N = K = 2048: 512 tiles for 2 x 256 resident workgroups;
// row-major operands 7% faster than the split 256 x 256 launch, row pairs 3%
// slower, taken on both so that the bits do not depend on the layout):
// 128 x 128 tiles instead, four times as many, two workgroups per CU, whole.
// p: the call's parameters with the 256 x 256 tile counts (replaced here).
static int launch_wgrad_small(WgradParams p, bool al16, hipStream_t st) {
  typedef CfgF8_128 Q;
  p.tiles_n = (int)cdiv(p.N, Q::BM);
  p.tiles_k = (int)cdiv(p.K, Q::BN);
  p.part = nullptr;
  p.dp = p.E * p.tiles_n * p.tiles_k;
  p.S = 1;
  p.units = 0;
  p.dev = 0;
  const dim3 grid((unsigned)(p.tiles_n * p.tiles_k), (unsigned)p.E);
  if (p.out_dtype == MXGG_DTYPE_BF16 && al16)
    hipLaunchKernelGGL((wgrad_kernel<Q, false, kEpiBf16>), grid, dim3(Q::NT), 0, st, p);
  else if (p.out_dtype == MXGG_DTYPE_F16 && al16)
    hipLaunchKernelGGL((wgrad_kernel<Q, false, kEpiF16>), grid, dim3(Q::NT), 0, st, p);
  else if (p.out_dtype == MXGG_DTYPE_F16)
    hipLaunchKernelGGL((wgrad_kernel<Q, false, kEpiF16Any>), grid, dim3(Q::NT), 0, st, p);
  else
    hipLaunchKernelGGL((wgrad_kernel<Q, false, kEpiAny>), grid, dim3(Q::NT), 0, st, p);
  return launch_status("wgrad");
}

// The plan of a wgrad call of `tiles` 256 x 256 tiles with `par` resident
// workgroups and `slots` partial-tile slots (0: no room): the host plan, and
// whether the kernels plan on the device and whether the call runs as 128 x
// 128 whole tiles instead (launch_wgrad_small).
struct WgradChoice {
  Split sp;
  bool dev;
  bool small;
};

static WgradChoice wgrad_choice(int E, int64_t M, int64_t N, int64_t K, int64_t tiles, int par, int slots) {
  constexpr int kib = CfgF8_256::BM * CfgF8_256::BN * 4 / 1024;
  WgradChoice w{split_plan((int)tiles, par, (int)wgrad_group_steps(E, M), slots, kib), false, false};
  // A lone round of several groups lasts as long as the longest group, which
  // only the device knows: the kernels plan from the groups' lengths
  // (wgrad_groups, or wgrad_plan past 64 groups) whenever a group of all M
  // rows would be split.
  w.dev = E > 1 && slots > 0 && split_plan((int)tiles, par, (int)cdiv(M, STEP) + 1, slots, kib).units > 0;
  const int64_t tiles128 = (int64_t)E * cdiv(N, 128) * cdiv(K, 128);
  w.small = (!w.dev && w.sp.units == 0 && 2 * tiles <= par) || (2 * tiles <= par && tiles128 >= 2 * par);
  return w;
}

// The wgrad launches of a checked call on step-major scales (gs: GO [T][N],
// is: IA [T][K] dwords); part / part_bytes: room for the fp32 partial tiles
// of tiles cut along the tokens (none: no tile is cut).  C: the 256 x 256
// configuration (XLine where GO, the X side, is row-major); the plan, the
// partial layout and the reduce are the one-stage configuration's, so both
// give the same bits.
template <class C>
static int launch_wgrad_c(const uint8_t* go_t, int64_t ld_go, const uint8_t* gs, const uint8_t* ia_t, int64_t ld_ia,
                          const uint8_t* is, const int32_t* offs, int E, int64_t M, int64_t N, int64_t K, void* out,
                          int out_dtype, int layout, void* part_area, size_t part_bytes, hipStream_t st) {
  const int64_t T = cdiv(M, STEP);
  // no more room than the split plans of this shape can use (ws_layout)
  const size_t cap = wgrad_part_cap(E, M, N, K);
  if (part_bytes > cap) part_bytes = cap;
  float* part = part_area && part_bytes ? (float*)part_area : nullptr;
  WgradParams p{go_t, ld_go, ia_t, ld_ia, gs, (uint32_t)(4 * T * N), is, (uint32_t)(4 * T * K), offs, E, M, N, K,
                (uint8_t*)out, out_dtype, (int)cdiv(N, C::BM), (int)cdiv(K, C::BN), part, 0, 1, 0, 0, 0, 0,
                (layout & MXGG_A_PAIRS) ? 1 : 0, (layout & MXGG_B_PAIRS) ? 1 : 0};
  const int64_t tiles = (int64_t)E * p.tiles_n * p.tiles_k;
  if (tiles > INT32_MAX / 2) return fail(MXGG_ERR_UNSUPPORTED, "wgrad: grid too large");
  static int resident_cache[64];
  const int par = resident_workgroups(wgrad_kernel<C, false>, C::NT, resident_cache);
  // groups differ in length, and with them the tiles' run times: with E > 1
  // only a lone under-filled round is split (its tiles all start at once)
  const bool may_split = E == 1 || tiles < par;
  const int slots = part && may_split ? split_slots<C>(part_bytes) : 0;
  const WgradChoice wc = wgrad_choice(E, M, N, K, tiles, par, slots);
  const Split& sp = wc.sp;
  p.dp = sp.dp;
  p.S = sp.S;
  p.units = sp.units;
  // device plan: the grids cover any such plan, every tile whole, or at most
  // min(par, slots) pieces and every tile reduced
  if (wc.dev) {
    p.dev = 1;
    p.par = par;
    p.slots = slots;
  }
  const bool al16 = K % 8 == 0 && (uintptr_t)out % 16 == 0;
  if (wc.small) return launch_wgrad_small(p, al16, st);
  const int64_t whole_ub = p.dev ? tiles : sp.dp;
  const int64_t units_ub = p.dev ? slots : sp.units;
  const int64_t split_tiles_ub = p.dev ? tiles : (sp.units ? sp.units / sp.S : 0);
  if (whole_ub > 0) {
    const dim3 grid((unsigned)(p.tiles_n * p.tiles_k), (unsigned)E);
    if (out_dtype == MXGG_DTYPE_BF16 && al16)
      hipLaunchKernelGGL((wgrad_kernel<C, false, kEpiBf16>), grid, dim3(C::NT), 0, st, p);
    else if (out_dtype == MXGG_DTYPE_F16 && al16)
      hipLaunchKernelGGL((wgrad_kernel<C, false, kEpiF16>), grid, dim3(C::NT), 0, st, p);
    else if (out_dtype == MXGG_DTYPE_F16)
      hipLaunchKernelGGL((wgrad_kernel<C, false, kEpiF16Any>), grid, dim3(C::NT), 0, st, p);
    else
      hipLaunchKernelGGL((wgrad_kernel<C, false, kEpiAny>), grid, dim3(C::NT), 0, st, p);
    if (int rc = launch_status("wgrad")) return rc;
  }
  if (units_ub <= 0) return MXGG_OK;
  hipLaunchKernelGGL((wgrad_kernel<C, true>), dim3((unsigned)units_ub), dim3(C::NT), 0, st, p);
  if (int rc = launch_status("wgrad")) return rc;
  hipLaunchKernelGGL((wgrad_reduce_kernel<StepCfg<C>>), dim3((unsigned)(split_tiles_ub * ReduceShape<C>::CH)),
                     dim3(256), 0, st, p);
  return launch_status("wgrad");
}

static int launch_wgrad(const uint8_t* go_t, int64_t ld_go, const uint8_t* gs, const uint8_t* ia_t, int64_t ld_ia,
                        const uint8_t* is, const int32_t* offs, int E, int64_t M, int64_t N, int64_t K, void* out,
                        int out_dtype, int layout, void* part_area, size_t part_bytes, hipStream_t st) {
  if (layout & MXGG_A_PAIRS)
    return launch_wgrad_c<CfgF8_256>(go_t, ld_go, gs, ia_t, ld_ia, is, offs, E, M, N, K, out, out_dtype, layout,
                                     part_area, part_bytes, st);
  return launch_wgrad_c<CfgF8_256X>(go_t, ld_go, gs, ia_t, ld_ia, is, offs, E, M, N, K, out, out_dtype, layout,
                                    part_area, part_bytes, st);
}

extern "C" int mxgg_wgrad_config(int E, int64_t M, int64_t N, int64_t K, int* block) {
  clear_error();
  if (!block) return fail(MXGG_ERR_INVALID_ARG, "wgrad_config: null output pointer");
  if (E <= 0 || E > 65535 || M < 0 || N <= 0 || K <= 0 || M > INT32_MAX || N > INT32_MAX || K > INT32_MAX)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad_config: shape out of range");
  typedef CfgF8_256 C;
  const int64_t tiles = (int64_t)E * cdiv(N, C::BM) * cdiv(K, C::BN);
  if (tiles > INT32_MAX / 2) return fail(MXGG_ERR_UNSUPPORTED, "wgrad_config: grid too large");
  if (int rc = require_device()) return rc;
  static int resident_cache[64];
  const int par = resident_workgroups(wgrad_kernel<C, false>, C::NT, resident_cache);
  if (par <= 0) return fail(MXGG_ERR_NO_DEVICE, "wgrad_config: resident workgroups unknown");
  const size_t part = wgrad_part_cap(E, M, N, K);
  const int slots = part && (E == 1 || tiles < par) ? split_slots<C>(part) : 0;
  *block = wgrad_choice(E, M, N, K, tiles, par, slots).small ? 128 : 256;
  return MXGG_OK;
}

extern "C" int mxgg_wgrad(const uint8_t* go_t, int64_t ld_go, const uint8_t* go_s, int64_t ld_gos,
                          const uint8_t* ia_t, int64_t ld_ia, const uint8_t* ia_s, int64_t ld_ias,
                          const int32_t* offs, int E, int64_t M, int64_t N, int64_t K, void* out,
                          int out_dtype, void* workspace, size_t ws_bytes, void* stream) {
  clear_error();
  bool empty;
  if (int rc = check_wgrad(go_t, ld_go, go_s, ld_gos, ia_t, ld_ia, ia_s, ld_ias, offs, E, M, N, K, out, out_dtype,
                           true, 0, &empty))
    return rc;
  if (empty) return MXGG_OK;
  const size_t need = wgrad_scale_bytes(M, N, K);
  if (need && (!workspace || ws_bytes < need))
    return fail(MXGG_ERR_WORKSPACE, "wgrad: workspace of at least %zu bytes needed, %zu given", need,
                workspace ? ws_bytes : (size_t)0);
  if (int rc = require_device()) return rc;
  hipStream_t st = (hipStream_t)stream;
  const int64_t T = cdiv(M, STEP);
  uint32_t* wsd = (uint32_t*)workspace;
  const WsLayout wl = ws_layout(ws_bytes, need, wgrad_part_cap(E, M, N, K));
  // Both operands in row pairs, staged at the end of the workspace from the
  // bytes past the partial area (ws_layout; 512 bytes of slack align both).
  const size_t stage = wgrad_staging_bytes(E, M, N, K);
  const bool staged = T > 0 && stage && wl.extra >= stage;
  PairJob pg{}, pi{};
  if (staged) {
    const int ldp = (int)staged_ld(M);
    uint8_t* dg = (uint8_t*)align256((size_t)((uint8_t*)workspace + ws_bytes - stage));
    uint8_t* di = (uint8_t*)align256((size_t)(dg + (size_t)N * ldp));
    pg = PairJob{go_t, ld_go, 0, dg, ldp, (int)(N / 2), 1, (int)M};
    pi = PairJob{ia_t, ld_ia, 0, di, ldp, (int)(K / 2), 1, (int)M};
  }
  if (T > 0) {
    if (int rc = launch_relayout(scale_job(go_s, ld_gos, 0, wsd, N, 1, M / 32, T),
                                 scale_job(ia_s, ld_ias, 0, wsd + T * N, K, 1, M / 32, T), st, "wgrad",
                                 staged ? &pg : nullptr, staged ? &pi : nullptr))
      return rc;
  }
  void* part = wl.part ? (void*)((uint8_t*)workspace + wl.part_off) : nullptr;
  return launch_wgrad(staged ? pg.dst : go_t, staged ? (int64_t)pg.ld_dst : ld_go, (const uint8_t*)wsd,
                      staged ? pi.dst : ia_t, staged ? (int64_t)pi.ld_dst : ld_ia, (const uint8_t*)(wsd + T * N), offs,
                      E, M, N, K, out, out_dtype, staged ? (MXGG_A_PAIRS | MXGG_B_PAIRS) : 0, part, wl.part, st);
}

extern "C" int mxgg_wgrad_steps(const uint8_t* go_t, int64_t ld_go, const uint32_t* go_ss, const uint8_t* ia_t,
                                int64_t ld_ia, const uint32_t* ia_ss, const int32_t* offs, int E, int64_t M,
                                int64_t N, int64_t K, void* out, int out_dtype, int layout, void* workspace,
                                size_t ws_bytes, void* stream) {
  clear_error();
  bool empty;
  if (int rc = check_wgrad(go_t, ld_go, (const uint8_t*)go_ss, 0, ia_t, ld_ia, (const uint8_t*)ia_ss, 0, offs, E, M,
                           N, K, out, out_dtype, false, layout, &empty))
    return rc;
  if (empty) return MXGG_OK;
  if (((uintptr_t)go_ss | (uintptr_t)ia_ss) & 3)
    return fail(MXGG_ERR_INVALID_ARG, "wgrad_steps: step-major scales must be 4-byte aligned");
  if (int rc = require_device()) return rc;
  return launch_wgrad(go_t, ld_go, (const uint8_t*)go_ss, ia_t, ld_ia, (const uint8_t*)ia_ss, offs, E, M, N, K, out,
                      out_dtype, layout, workspace, workspace ? ws_bytes : 0, (hipStream_t)stream);
}
