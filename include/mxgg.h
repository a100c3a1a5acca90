/*
 * mxgg.h -- C ABI of the MI355X (gfx950) MX-scaled grouped-GEMM library
 * (libmxgg.so).
 *
 * Plain pointers, sizes and strides only.  Every pointer argument named *_ptr
 * or out* is a device pointer; `stream` is a hipStream_t passed as void*
 * (NULL = the default stream).  No entry point allocates device memory, frees
 * it or synchronises the stream: callers own every buffer, and all work is
 * enqueued on `stream` in order.
 *
 * Return value: 0 on success, a negative MXGG_ERR_* for an argument that was
 * rejected before anything was launched, a positive hipError_t when the HIP
 * runtime refused a launch.  mxgg_last_error_string() describes the most recent
 * failure on the calling thread.
 *
 * Data formats (the reference's `to_mx` layout, utils.py:67-105):
 *   e4m3   one byte per element (float8_e4m3fn)
 *   e2m1   two elements per byte, element 2i in the low nibble
 *   scales one e8m0 byte per 32 consecutive elements of the quantized
 *          (contiguous) dimension, value 2**(s-127), plain row-major layout
 *          (rows, cols/32) with a row stride.
 * Strides are in ELEMENTS of the pointed-to tensor (bytes for e4m3 and scale
 * tensors, bytes -- i.e. element pairs -- for packed e2m1 tensors).
 *
 * Step-major scales (MXGG_SCALES_STEPS), the layout the GEMM kernels read:
 * for an operand of `batch` matrices of R rows whose rows hold nblk scale
 * bytes, T = ceil(nblk / 4) and dword (b, t, r) -- uint32 index
 * (b*T + t)*R + r -- holds blocks 4t .. 4t+3 of row r of matrix b, block
 * 4t+j in byte j; bytes past nblk are 127 (2**0).  The quantizers write it on
 * request, and the *_steps GEMM entry points take it, skipping the per-call
 * re-layout of plain scales.  (Not the reference's CDNA4 pre-shuffle,
 * kernels/forward.py:367-397: one 128-element step of a row is one dword.)
 *
 * Row-pair data (MXGG_DATA_PAIRS for the quantizers, MXGG_A_PAIRS /
 * MXGG_B_PAIRS for the *_steps GEMMs; no counterpart in the reference, whose
 * operands are row-major): an e4m3 operand of R rows (R even) whose rows hold
 * L bytes, with "row stride" ld >= L rounded up to 64, keeps byte k of row r
 * at (r/2)*2*ld + (k/64)*128 + (r%2)*64 + k%64.  The 64-byte pieces of rows 2i
 * and 2i+1 alternate, so the 64-element slice of two adjacent rows that the
 * GEMM stages per step is one 128-byte line (row-major, each is half of two
 * lines).  Bytes L .. L rounded up to 64 of a row are padding, which the
 * GEMMs do not read (they take the true K, resp. M); the quantizers write
 * zeros there.  Row quads (MXGG_DATA_QUADS, MXGG_B_QUADS) are the same for
 * packed e2m1 data, whose 64-element stage piece of a row is 32 bytes: 4 rows
 * (R divisible by 4) interleave in 32-byte pieces, byte k of row r at
 * (r/4)*4*ld + (k/32)*128 + (r%4)*32 + k%32, ld = the row's bytes rounded up
 * to 32.
 */
#ifndef MXGG_H_
#define MXGG_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXGG_VERSION 4001 /* major*1000 + minor */

/* status codes */
#define MXGG_OK 0
#define MXGG_ERR_INVALID_ARG (-1)   /* bad shape, stride, alignment or enum */
#define MXGG_ERR_UNSUPPORTED (-2)   /* valid request this build does not implement */
#define MXGG_ERR_WORKSPACE (-3)     /* workspace missing or too small */
#define MXGG_ERR_NO_DEVICE (-4)     /* no gfx950 device current */

/* element formats (codes match the f8f6f4 MFMA cbsz/blgp encoding) */
#define MXGG_FMT_E4M3 0
#define MXGG_FMT_E2M1 4

/* host element types for quantizer inputs and GEMM outputs */
#define MXGG_DTYPE_BF16 0
#define MXGG_DTYPE_F16 1
#define MXGG_DTYPE_F32 2

/* scale layouts of the quantizer outputs, and the data-layout flag OR-ed
 * into the same argument */
#define MXGG_SCALES_PLAIN 0   /* (rows, nblk) bytes, row stride ld_s */
#define MXGG_SCALES_STEPS 1   /* step-major dwords (see above); ld_s = R, the rows per batch */
#define MXGG_DATA_PAIRS 2     /* e4m3 data outputs in row pairs (see above) */
#define MXGG_DATA_QUADS 4     /* packed e2m1 data outputs in row quads (see above) */

/* operand layouts of mxgg_grouped_mm_steps / mxgg_wgrad_steps (bit flags;
 * 0 = both row-major) */
#define MXGG_A_PAIRS 1   /* A (forward) or go_t (wgrad) in row pairs */
#define MXGG_B_PAIRS 2   /* B (forward; e4m3 only) or ia_t (wgrad) in row pairs */
#define MXGG_B_QUADS 4   /* B (forward; packed e2m1 only) in row quads */

/* Library version (MXGG_VERSION of the build). */
int mxgg_version(void);

/* Message for the last failure on this thread ("" if none). */
const char* mxgg_last_error_string(void);

/* 1 if the current HIP device is a gfx950 part the kernels were built for,
 * 0 otherwise.  Replaces `_rocm_mxfp8_available` (kernels/_common.py:27) and
 * `is_MI350` (utils.py:108-115). */
int mxgg_device_supported(void);

/*
 * MX quantization along the contiguous last dimension (FLOOR scale mode).
 * Replaces `to_mx(data, elem_dtype, block_size=32)` (utils.py:67-105).
 *   src        (rows, cols) of src_dtype, row stride ld_src elements
 *   elem_fmt   MXGG_FMT_E4M3 (q is (rows, cols) bytes, row stride ld_q) or
 *              MXGG_FMT_E2M1 (q is (rows, cols/2) packed bytes, row stride ld_q)
 *   scales     scale_layout MXGG_SCALES_PLAIN: (rows, cols/32) bytes, row stride
 *              ld_s.  MXGG_SCALES_STEPS: step-major for batches of ld_s rows
 *              (ld_s divides rows; e.g. ld_s = N for an (E, N, K) weight
 *              given as E*N rows), 4 * rows * ceil(cols/128) bytes.
 *   scale_layout | MXGG_DATA_PAIRS: q in row pairs (E4M3, rows even, ld_q a
 *              multiple of 64 and at least cols rounded up to 64);
 *              | MXGG_DATA_QUADS: q in row quads (E2M1, rows divisible by 4,
 *              ld_q a multiple of 32 and at least cols/2 rounded up to 32).
 * cols must be a multiple of 32.
 */
int mxgg_quantize_mx(const void* src, int src_dtype, int64_t rows, int64_t cols,
                     int64_t ld_src, int elem_fmt, void* q, int64_t ld_q,
                     uint8_t* scales, int64_t ld_s, int scale_layout, void* stream);

/*
 * MX quantization along dimension 0 with a transposed output: the result is
 * exactly to_mx(src.t().contiguous()) -- the "dim1-quantized" operands the
 * weight gradient takes (kernels/backward.py:232-243).
 *   src     (rows, cols) of src_dtype, row stride ld_src; rows % 32 == 0
 *   q       (cols, rows) e4m3 bytes, row stride ld_q (elem_fmt must be E4M3)
 *   scales  MXGG_SCALES_PLAIN: (cols, rows/32) bytes, row stride ld_s;
 *           MXGG_SCALES_STEPS: step-major [ceil(rows/128)][cols] dwords (ld_s = cols)
 *   scale_layout | MXGG_DATA_PAIRS: q in row pairs (cols even, ld_q a multiple
 *           of 64 and at least rows rounded up to 64)
 */
int mxgg_quantize_mx_dim0(const void* src, int src_dtype, int64_t rows, int64_t cols,
                          int64_t ld_src, int elem_fmt, void* q, int64_t ld_q,
                          uint8_t* scales, int64_t ld_s, int scale_layout, void* stream);

/*
 * Both MX layouts from one read of src: q_rows / s_rows = to_mx(src) and
 * q_cols / s_cols = to_mx(src.t().contiguous()), e4m3, for `batch` stacked
 * (rows, cols) matrices (batch stride rows * ld_src elements; outputs stacked
 * the same way).  The fused cast-transpose step the reference's callers need
 * for the backward pass: a gradient quantized along N for dgrad and along M
 * for wgrad (kernels/backward.py:232-233), or an expert weight (E, N, K)
 * quantized along K for the forward and along N, transposed to (E, K, N),
 * for dgrad (kernels/forward.py:485-488).  Bit-identical to mxgg_quantize_mx
 * + mxgg_quantize_mx_dim0.
 *   src     (batch, rows, cols) of src_dtype, row stride ld_src; rows % 32 == 0, cols % 32 == 0
 *   q_rows  (batch, rows, cols) e4m3, row stride ld_qr;  s_rows (batch, rows, cols/32), row stride ld_sr
 *   q_cols  (batch, cols, rows) e4m3, row stride ld_qc;  s_cols (batch, cols, rows/32), row stride ld_sc
 *   scale_layout MXGG_SCALES_STEPS: s_rows is [batch][ceil(cols/128)][rows] and s_cols
 *           [batch][ceil(rows/128)][cols] dwords (ld_sr = rows, ld_sc = cols)
 *   scale_layout | MXGG_DATA_PAIRS: q_rows and q_cols in row pairs (ld_qr, ld_qc
 *           multiples of 64, at least cols, resp. rows, rounded up to 64)
 */
int mxgg_quantize_mx_both(const void* src, int src_dtype, int64_t batch, int64_t rows, int64_t cols,
                          int64_t ld_src, void* q_rows, int64_t ld_qr, uint8_t* s_rows, int64_t ld_sr,
                          void* q_cols, int64_t ld_qc, uint8_t* s_cols, int64_t ld_sc, int scale_layout,
                          void* stream);

/*
 * Routing table of the grouped GEMM, in the reference's buffer format
 * [hist E | start E | total 1 | map grid_m_ub] (int32), where
 * grid_m_ub = cdiv(M, block_m) + max(E-1, 0) and map[p] = (block << 16) | e or -1.
 * Replaces `_build_expt_data` / `_expt_data_kernel` (kernels/forward.py:296-365).
 * The GEMMs build no such buffer: every workgroup looks its tile up from offs.
 * This test hook fills the reference's buffer with that same lookup
 * (route_tile with one column tile and bands of one m-block, whose order is
 * the reference's m-block order).  out must hold mxgg_routing_words() int32s.
 */
int64_t mxgg_routing_words(int E, int64_t M, int block_m);
int mxgg_build_routing(const int32_t* offs, int E, int64_t M, int block_m, int32_t* out,
                       void* stream);

/*
 * Tile order of the forward / dgrad GEMM (test hook): for every program id p
 * of the whole-tile launch grid (mxgg_schedule_programs() programs) writes
 * the tile the kernel computes there, out[5p .. 5p+4] = (expert, row0, rows,
 * n0, cols), or five -1s for programs that exit.  It runs the kernel's own
 * routing code: the XCD swizzle of the reference (kernels/forward.py:31-36),
 * then expert-aligned GROUP_M bands -- the tiles of each group contiguous,
 * cut into bands of at most group_m m-blocks, column-major inside a band --
 * in place of the reference's bands over the global m-block index
 * (kernels/forward.py:38-51, 111-127).  block_m x block_n must be a built
 * tile (256 x 256 or 128 x 128).
 */
int64_t mxgg_schedule_programs(int E, int64_t M, int64_t N, int block_m, int block_n);
int mxgg_tile_schedule(const int32_t* offs, int E, int64_t M, int64_t N, int block_m,
                       int block_n, int group_m, int xcd_swizzle, int32_t* out, void* stream);

/*
 * Launch configuration the library uses for a grouped GEMM of this shape:
 * tile (block_m x block_n; the reduction step is fixed at 128), GROUP_M and
 * XCD swizzle width.  Requests (nonzero *block_m, *block_n, *group_m,
 * *xcd_swizzle on entry) are applied as mxgg_grouped_mm applies them; the
 * call returns MXGG_ERR_UNSUPPORTED when the resulting tile is not built.
 * Replaces `_pick_config` / `_BEST_CFGS` / `_FALLBACK_*`
 * (kernels/forward.py:399-459).  The answer is the one for a
 * mxgg_grouped_mm call given room to stage its operands (the drop-in call):
 * a tuned entry's GROUP_M and XCD swizzle apply only to calls on the operand
 * layout it was timed on, so a *_steps call on another layout may get the
 * built-in order (tile shape and split stay the entry's: same bits).
 */
int mxgg_grouped_mm_config(int E, int64_t M, int64_t N, int64_t K, int b_fmt, int* block_m,
                           int* block_n, int* group_m, int* xcd_swizzle);

/*
 * Forward / dgrad grouped GEMM: out[s:e, :] = A[s:e, :] @ B[g]^T for each group
 * g with rows [offs[g-1], offs[g]) (offs[-1] = 0), MX scales applied per 32
 * elements of K, fp32 accumulation, one rounding to out_dtype.
 * Replaces `triton_mxfp8_grouped_mm` (kernels/forward.py:461-606).
 *   A        (M, K) e4m3, row stride lda
 *   A_s      (M, K/32) scales, row stride ldas
 *   B        (E, N, K) in b_fmt: e4m3 (row stride ldb_n >= K) or e2m1 packed
 *            (row stride ldb_n >= K/2), expert stride ldb_e
 *   B_s      (E, N, K/32) scales, row stride ldbs_n, expert stride ldbs_e
 *   offs     (E,) int32 cumulative group ends, device memory, nondecreasing,
 *            offs[E-1] <= M
 *   out      (M, N) of out_dtype, row stride ldo.  Rows >= offs[E-1] are not
 *            written (as in the reference).
 *   block_m, block_n, group_m, xcd_swizzle: 0 = library choice; otherwise a
 *            request honoured when the build has that tile shape.
 *   workspace / ws_bytes: device scratch, contents need not be initialised
 *            and are overwritten.  Required: 4 * ceil(K/128) * (M + E*N) bytes,
 *            the scales re-laid step-major for the kernel (the reference re-lays
 *            them per call too, kernels/forward.py:537-550).  Recommended:
 *            mxgg_grouped_mm_workspace_size(E, M, N, K) bytes, which adds (after
 *            the scales, 256-byte aligned) room for the fp32 partial tiles of a
 *            last, partial round of tiles cut along K (at most 128 MiB; only for
 *            K >= 4096 and short launches).  With less, fewer or no tiles are
 *            cut; more room than that is not used for partial tiles.  Bytes
 *            past the scales and that partial room hold the staged operands:
 *            with at least mxgg_grouped_mm_staging_size(E, M, N, K, b_fmt) of
 *            them, an e4m3 B and / or A is first copied into row pairs at the
 *            end of the workspace (in the scale re-layout launch), which the
 *            GEMM reads in whole 128-byte lines.  A workspace of exactly the
 *            recommended size stages nothing; staging never takes room from the
 *            partial tiles, and the output bits are the same either way.
 *            A call that stages nothing, of at most 1.2e11 flop (2*M*N*K), on
 *            scales whose rows and expert strides are 16-byte multiples at
 *            16-byte aligned addresses, reads the plain scales directly (no
 *            re-layout launch; the scale room of the workspace is still
 *            required and left unused): the same bits.
 * K must be a multiple of 32.  A and B rows must be 16-byte aligned; scale
 * rows need no alignment.  Results do not depend on the workspace size beyond
 * fp32 summation order (a cut tile adds its pieces in a fixed order, so
 * repeated calls give identical bits).
 */
size_t mxgg_grouped_mm_workspace_size(int E, int64_t M, int64_t N, int64_t K);
/*
 * Workspace bytes, on top of mxgg_grouped_mm_workspace_size, with which
 * mxgg_grouped_mm stages e4m3 operands in row pairs, or 0 where the copies
 * would not pay for themselves: B (E * N * K rounded up to 64, plus 256) for
 * E <= M / 8192 and K >= 4096, or K >= 2048 with N >= 4096 (e4m3 B only); A
 * (M * K rounded up to 64, plus 256) for N >= 8192, K >= 2048, M even and
 * M * N * K above 6e10 (e4m3 or e2m1 B; smaller calls skip the re-layout
 * launch instead, see mxgg_grouped_mm).  The copies then
 * cost a few percent of the GEMM's time and save more.  No counterpart in the
 * reference, whose Triton kernel reads its operands where they lie.
 */
size_t mxgg_grouped_mm_staging_size(int E, int64_t M, int64_t N, int64_t K, int b_fmt);
int mxgg_grouped_mm(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas,
                    const uint8_t* B, int b_fmt, int64_t ldb_n, int64_t ldb_e,
                    const uint8_t* B_s, int64_t ldbs_n, int64_t ldbs_e,
                    const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                    void* out, int out_dtype, int64_t ldo,
                    int block_m, int block_n, int group_m, int xcd_swizzle,
                    void* workspace, size_t ws_bytes, void* stream);

/*
 * mxgg_grouped_mm with step-major scales (MXGG_SCALES_STEPS, written so by the
 * quantizers): A_ss [T][M] and B_ss [E][T][N] uint32, T = ceil(K/128).  The
 * same GEMM launches without the per-call re-layout of plain scales (the
 * reference pre-shuffles its scales on every call too, kernels/forward.py:
 * 367-397, 528-550).  layout: MXGG_A_PAIRS and / or MXGG_B_PAIRS for operands
 * in row pairs (lda, ldb_n then at least K rounded up to 64; M, resp. N,
 * even), MXGG_B_QUADS for a packed e2m1 B in row quads (ldb_n at least K/2
 * rounded up to 32, N divisible by 4).  workspace / ws_bytes (may be null / 0): room for
 * the fp32 partial tiles of a split last round;
 * mxgg_grouped_mm_workspace_size() is always enough.  Results are
 * bit-identical to mxgg_grouped_mm given a workspace with the same room after
 * its scales, in either operand layout.
 */
int mxgg_grouped_mm_steps(const uint8_t* A, int64_t lda, const uint32_t* A_ss,
                          const uint8_t* B, int b_fmt, int64_t ldb_n, int64_t ldb_e, const uint32_t* B_ss,
                          const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                          void* out, int out_dtype, int64_t ldo,
                          int block_m, int block_n, int group_m, int xcd_swizzle, int layout,
                          void* workspace, size_t ws_bytes, void* stream);

/*
 * mxgg_grouped_mm without a workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  Same arguments,
 * results and errors as mxgg_grouped_mm given a workspace of
 * MXGG_NOALLOC_SCRATCH_BYTES bytes (operands are staged only where the
 * scales, the full partial room and the staging all fit in it); the
 * workspace is instead a device array
 * inside this library, one per GPU, allocated when the library is loaded and
 * held until the process ends.  Calls it cannot take -- the re-laid scales,
 * 4 * ceil(K/128) * (M + E*N) bytes, above MXGG_NOALLOC_SCRATCH_BYTES -- are
 * rejected with MXGG_ERR_WORKSPACE before anything is launched.  The call
 * itself allocates nothing.  Every call on a GPU uses that GPU's one array:
 * calls that overlap on one GPU (other streams, other threads) race and give
 * wrong results; serialise them.
 */
#define MXGG_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)
int mxgg_grouped_mm_noalloc(const uint8_t* A, int64_t lda, const uint8_t* A_s, int64_t ldas,
                            const uint8_t* B, int b_fmt, int64_t ldb_n, int64_t ldb_e,
                            const uint8_t* B_s, int64_t ldbs_n, int64_t ldbs_e,
                            const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                            void* out, int out_dtype, int64_t ldo,
                            int block_m, int block_n, int group_m, int xcd_swizzle, void* stream);

/*
 * Weight-gradient grouped GEMM: out[g] = GO[:, s:e] @ IA[:, s:e]^T, shape (E, N, K),
 * a reduction over each group's token range; an empty group gives zeros.
 * Replaces `triton_mxfp8_wgrad` (kernels/backward.py:217-305), including its
 * store of bf16-rounded values whatever out_dtype is (backward.py:101-104,
 * 214, 251): f32 holds the bf16 value, f16 the bf16 value converted (RNE).
 *   go_t  (N, M) e4m3, row stride ld_go;   go_s (N, M/32), row stride ld_gos
 *   ia_t  (K, M) e4m3, row stride ld_ia;   ia_s (K, M/32), row stride ld_ias
 *   offs  (E,) int32 cumulative group ends, nondecreasing, offs[E-1] <= M.
 *         Any values: as in the reference (token masks by group, scales by
 *         token / 32), a 32-token scale block shared by two groups scales the
 *         tokens of both.
 *   out   (E, N, K) of out_dtype (BF16, F16 or F32), contiguous
 *   workspace / ws_bytes: device scratch, need not be initialised.  Required:
 *         4 * ceil(M/128) * (N + K) bytes (the scales re-laid step-major);
 *         recommended: mxgg_wgrad_workspace_size(E, M, N, K), which adds room
 *         for the fp32 partial tiles of tiles cut along the token range when
 *         the tiles do not fill the chip (E = 1, or fewer tiles than
 *         resident workgroups; with E > 1 sized for a group of all M tokens,
 *         since the kernels cut by the longest group), at most 128 MiB; more
 *         is not used for partial tiles.  With mxgg_wgrad_staging_size(E, M,
 *         N, K) bytes past the scales and that room, go_t and ia_t are first
 *         copied into row pairs at the end of the workspace (in the scale
 *         re-layout launch) and the GEMM reads whole 128-byte lines of them;
 *         the recommended size alone stages nothing, the partial tiles keep
 *         their room, and the output bits are the same either way.
 */
size_t mxgg_wgrad_workspace_size(int E, int64_t M, int64_t N, int64_t K);
/*
 * Workspace bytes, on top of mxgg_wgrad_workspace_size, with which mxgg_wgrad
 * stages both operands in row pairs ((N + K) * M rounded up to 64, plus 512),
 * or 0 where the copy would not pay for itself: it is offered only for N and
 * K both at least 8192, or with E >= 8 groups for N + K >= 10240 (elsewhere
 * the GEMM reads row-major go_t in whole lines, XLine), and never for odd N
 * or K or for M not a multiple of 32.  No counterpart in the reference.
 */
size_t mxgg_wgrad_staging_size(int E, int64_t M, int64_t N, int64_t K);
/*
 * Tile edge (256 or 128, into *block) of the GEMM launches of a mxgg_wgrad /
 * mxgg_wgrad_steps call of this shape given the recommended workspace
 * (mxgg_wgrad_workspace_size): 128 x 128 tiles where 256 x 256 tiles would
 * fill at most half the chip and either no tile of them is cut along the
 * tokens or 128 x 128 tiles fill at least one round; else 256 x 256.  Reads
 * the device's resident workgroup count (MXGG_ERR_NO_DEVICE without one).
 * Replaces the tile and split choice of `triton_mxfp8_wgrad`
 * (kernels/backward.py:245-254), as mxgg_grouped_mm_config does the
 * forward's.
 */
int mxgg_wgrad_config(int E, int64_t M, int64_t N, int64_t K, int* block);
int mxgg_wgrad(const uint8_t* go_t, int64_t ld_go, const uint8_t* go_s, int64_t ld_gos,
               const uint8_t* ia_t, int64_t ld_ia, const uint8_t* ia_s, int64_t ld_ias,
               const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
               void* out, int out_dtype, void* workspace, size_t ws_bytes, void* stream);

/*
 * mxgg_wgrad with step-major scales: go_ss [T][N] and ia_ss [T][K] uint32,
 * T = ceil(M/128) (mxgg_quantize_mx_dim0 / _both with MXGG_SCALES_STEPS), no
 * re-layout.  layout: MXGG_A_PAIRS (go_t) and / or MXGG_B_PAIRS (ia_t) for
 * operands in row pairs (ld_go, ld_ia then at least M rounded up to 64; N,
 * resp. K, even).  workspace / ws_bytes (may be null / 0): room for the fp32
 * partial tiles of tiles cut along the tokens; mxgg_wgrad_workspace_size() is
 * always enough.  Bit-identical to mxgg_wgrad given the same room, in either
 * operand layout.
 */
int mxgg_wgrad_steps(const uint8_t* go_t, int64_t ld_go, const uint32_t* go_ss,
                     const uint8_t* ia_t, int64_t ld_ia, const uint32_t* ia_ss,
                     const int32_t* offs, int E, int64_t M, int64_t N, int64_t K,
                     void* out, int out_dtype, int layout, void* workspace, size_t ws_bytes,
                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXGG_H_ */
