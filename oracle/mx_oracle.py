"""CPU oracle for the MX-scaled grouped-GEMM hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the ``kernels`` package, the
``utils`` drop-in module or the HIP library) imports this module; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
use it, and only as the checker / the timed CPU baseline.

Every function restates, in numpy (and plain Python loops where the inputs are
tiny), one piece of the reference's algorithm.  The reference file:line each
function follows is cited in its docstring.  How each function is pinned
(golden vectors, closed forms, brute force, torch's own cast routine) is listed
in ``PINNING`` at the bottom of this file and exercised by
``tests/test_oracle.py``.

Conventions
-----------
* bf16 tensors are carried as ``uint16`` bit patterns (numpy has no bf16).
* e4m3 (float8_e4m3fn) tensors are carried as ``uint8`` codes.
* e2m1 tensors are carried packed two per byte, element ``2i`` in the low
  nibble (torch ``Float4_e2m1fn_x2`` convention).
* e8m0 scales are ``uint8`` biased exponents (value ``2**(s-127)``).
"""

from __future__ import annotations

import math
import random as _random

import numpy as np

E4M3_MAX = 448.0
F8E4M3_MAX_POW2 = 8      # floor(log2(448)); utils.py:63-64
E2M1_MAX = 6.0
F4E2M1_MAX_POW2 = 2      # floor(log2(6)); OCP MX v1.0 FP4 (e2m1) emax
BLOCK = 32

# ----------------------------------------------------------------------------
# bit-level helpers
# ----------------------------------------------------------------------------


def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns to float32."""
    u16 = np.asarray(u16, dtype=np.uint16)
    return (u16.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round-to-nearest-even; every NaN becomes 0x7FC0.

    Restates torch's ``round_to_nearest_even`` (c10/util/BFloat16.h), which is
    what ``acc.to(torch.bfloat16)`` / Triton's bf16 store do for finite values
    (kernels/forward.py:293, kernels/backward.py:103).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    r[np.isnan(x)] = 0x7FC0
    return r


# e4m3fn decode table (OCP FP8 E4M3: bias 7, no inf, 0x7F/0xFF = NaN)
def _build_e4m3_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 7
        if e == 0xF and m == 7:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * m * 2.0 ** -9
        else:
            t[c] = s * (1 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_TABLE = _build_e4m3_table()

# e2m1 decode table (OCP FP4 E2M1: bias 1, no inf / NaN)
E2M1_TABLE = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                       -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)


def e4m3_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> e4m3fn code, round-to-nearest-even.

    Behaviour of torch's ``Tensor.to(torch.float8_e4m3fn)`` (used at
    utils.py:102): RNE onto the e4m3 grid (subnormal step 2**-9), the sign kept
    for zeros, and every |x| >= 480 (and NaN / inf) mapped to the NaN code 0x7F
    with the sign bit OR-ed in.  Written from the format definition, not from
    torch's bit tricks; ``tests/test_oracle.py`` checks it against torch's own
    cast over every bf16 bit pattern and their fp32 neighbours.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> np.uint32(24)) & np.uint32(0x80)).astype(np.uint8)
    with np.errstate(invalid="ignore"):      # signalling-NaN bit patterns
        a = np.abs(x.astype(np.float64))
        big = ~(a < 480.0)                   # also catches NaN and inf
    a = np.where(big, 0.0, a)
    _, ex = np.frexp(a)                      # a = m * 2**ex, m in [0.5, 1)
    e = np.maximum(ex - 1, -6)               # exponent of the e4m3 binade (subnormals use -6)
    ulp = np.ldexp(1.0, e - 3)
    q = np.rint(a / ulp)                     # numpy rint = round half to even; exact division
    code = ((e + 6) * 8 + q).astype(np.int64)
    code = np.where(a == 0.0, 0, code)
    code = np.where(big, 0x7F, code)
    return (code.astype(np.uint8) | sign)


def e2m1_from_f32(x: np.ndarray) -> np.ndarray:
    """float32 -> e2m1 nibble (0..15), round-to-nearest-even, saturating.

    OCP MX v1.0 FP4 conversion as used by torchao's MX FLOOR recipe for fp4
    (the reference has no fp4 path; utils.py:78 asserts e4m3).  Values beyond 6
    saturate to +-6; NaN maps to the max-magnitude code with the NaN's sign
    (e2m1 has no NaN; the spec leaves this implementation-defined).
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> np.uint32(28)) & np.uint32(0x8)).astype(np.uint8)
    with np.errstate(invalid="ignore"):
        a = np.abs(x.astype(np.float64))
    nan = np.isnan(a)
    a = np.where(nan, 6.0, np.minimum(a, 6.0))
    _, ex = np.frexp(a)
    e = np.maximum(ex - 1, 0)                # binade exponent; subnormal binade uses 0
    ulp = np.ldexp(1.0, e - 1)               # one mantissa bit
    q = np.rint(a / ulp)                     # 0..4 within the binade (carry ok)
    code = (e * 2 + q).astype(np.int64)
    code = np.where(a == 0.0, 0, code)
    code = np.minimum(code, 7)
    return code.astype(np.uint8) | sign


def pack_e2m1(nibbles: np.ndarray) -> np.ndarray:
    """Pack nibbles along the last dim: byte i = n[2i] | n[2i+1] << 4."""
    n = np.asarray(nibbles, dtype=np.uint8)
    return (n[..., 0::2] | (n[..., 1::2] << 4)).astype(np.uint8)


def unpack_e2m1(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


# ----------------------------------------------------------------------------
# quantizer (to_mx, FLOOR mode)
# ----------------------------------------------------------------------------


def _as_f32(x, src: str) -> np.ndarray:
    if src == "bf16":
        return bf16_bits_to_f32(x)
    if src in ("f32", "f16"):
        return np.asarray(x).astype(np.float32)
    raise ValueError(src)


def mx_scales(blocks_f32: np.ndarray, max_pow2: int) -> np.ndarray:
    """e8m0 FLOOR scale per block (last axis = the 32 block elements).

    utils.py:86-95: amax in the input dtype (NaN-propagating), widened to fp32,
    clamped below at fp32 tiny, biased exponent field e = bits[30:23], stored
    scale = clamp(e - 127 - max_pow2 + 127, 0, 254).
    """
    amax = np.max(np.abs(blocks_f32), axis=-1)          # NaN propagates like torch.amax
    amax = np.where(np.isnan(amax), amax, np.maximum(amax, np.float32(np.finfo(np.float32).tiny)))
    e = ((amax.astype(np.float32).view(np.uint32) >> np.uint32(23)) & np.uint32(0xFF)).astype(np.int64)
    return np.clip(e - max_pow2, 0, 254).astype(np.uint8)


def to_mx(x, src: str = "bf16", elem: str = "e4m3", block: int = BLOCK):
    """Quantize along the last dim; returns ``(scales_u8, data)``.

    Follows utils.py:67-105 (``to_mx``): per ``block``-element group, FLOOR e8m0
    scale (``mx_scales``), then ``clamp(x / 2**(s-127), +-max)`` cast to the
    element format.  Dividing by the power of two ``2**(s-127)`` is done as the
    exact multiplication by ``2**(127-s)``.  ``elem='e4m3'`` returns e4m3 codes of
    the input's shape; ``elem='e2m1'`` returns packed nibbles with a last dim
    half as long (max_pow2 = 2, saturation at 6).
    """
    xf = _as_f32(x, src)
    if xf.shape[-1] % block:
        raise AssertionError(f"last dim {xf.shape[-1]} must be divisible by block_size {block}")
    shp = xf.shape
    xb = xf.reshape(-1, shp[-1] // block, block)
    max_pow2 = F8E4M3_MAX_POW2 if elem == "e4m3" else F4E2M1_MAX_POW2
    s = mx_scales(xb, max_pow2)
    mul = np.ldexp(np.float32(1.0), (127 - s.astype(np.int32))).astype(np.float32)  # 2**(127-s), exact
    with np.errstate(invalid="ignore"):      # NaN inputs (signalling patterns)
        scaled = xb * mul[..., None]
    lim = np.float32(E4M3_MAX if elem == "e4m3" else E2M1_MAX)
    scaled = np.where(np.isnan(scaled), scaled, np.clip(scaled, -lim, lim))
    if elem == "e4m3":
        q = e4m3_from_f32(scaled).reshape(shp)
    elif elem == "e2m1":
        q = pack_e2m1(e2m1_from_f32(scaled).reshape(shp))
    else:
        raise ValueError(elem)
    return s.reshape(shp[:-1] + (shp[-1] // block,)), q


def step_major(scales: np.ndarray) -> np.ndarray:
    """Plain scales ``(..., R, nblk)`` (uint8) -> the build's step-major layout
    ``(..., T, R)`` uint32, ``T = cdiv(nblk, 4)``: word ``[t, r]`` holds
    blocks ``4t .. 4t+3`` of row r, block ``4t+j`` in byte j, bytes past nblk
    127.  Not the reference's CDNA4 pre-shuffle (kernels/forward.py:367-397);
    the layout the build's GEMM kernels read and its quantizers can write.
    """
    s = np.asarray(scales, dtype=np.uint8)
    nblk = s.shape[-1]
    T = -(-nblk // 4)
    pad = np.full(s.shape[:-1] + (4 * T,), 127, dtype=np.uint8)
    pad[..., :nblk] = s
    words = pad.reshape(s.shape[:-1] + (T, 4)).astype(np.uint32)
    w = words[..., 0] | (words[..., 1] << 8) | (words[..., 2] << 16) | (words[..., 3] << 24)
    return np.swapaxes(w, -1, -2).copy()


def plain_from_step_major(words: np.ndarray, nblk: int) -> np.ndarray:
    """Inverse of ``step_major``: ``(..., T, R)`` uint32 -> ``(..., R, nblk)`` uint8."""
    w = np.swapaxes(np.asarray(words, dtype=np.uint32), -1, -2)
    b = np.stack([(w >> (8 * j)) & 0xFF for j in range(4)], axis=-1).astype(np.uint8)
    return b.reshape(w.shape[:-1] + (4 * w.shape[-1],))[..., :nblk].copy()


def dequant(q: np.ndarray, scales: np.ndarray, elem: str = "e4m3", block: int = BLOCK,
            dtype=np.float64) -> np.ndarray:
    """Dequantize along the last dim: value * 2**(s-127) (exact in fp32/fp64).

    The math the scaled dot computes per block (kernels/forward.py:238-240,
    kernels/backward.py:94-98; the ``tl.dot_scaled`` semantics).
    """
    if elem == "e4m3":
        v = E4M3_TABLE[np.asarray(q, dtype=np.uint8)].astype(dtype)
    elif elem == "e2m1":
        v = E2M1_TABLE[unpack_e2m1(q)].astype(dtype)
    else:
        raise ValueError(elem)
    sh = v.shape
    vb = v.reshape(sh[:-1] + (sh[-1] // block, block))
    f = np.ldexp(np.ones(scales.shape, dtype=dtype), np.asarray(scales, dtype=np.int32) - 127)
    return (vb * f[..., None]).reshape(sh)


# ----------------------------------------------------------------------------
# offsets, routing table, tile schedule
# ----------------------------------------------------------------------------


def generate_jagged_offs(E: int, M: int, multiple_of: int = 32, rng: _random.Random | None = None) -> np.ndarray:
    """Random sorted cumulative group-end offsets, multiples of ``multiple_of``, last = M.

    utils.py:35-50: E-1 distinct values from {m, 2m, ..., M-m} via
    ``random.sample``, plus M, sorted.  ``rng`` defaults to the module-level
    ``random`` state, as in the reference.
    """
    if M % multiple_of != 0:
        raise ValueError(f"M must be divisible by {multiple_of}")
    possible = list(range(multiple_of, M + 1, multiple_of))
    if E > len(possible):
        raise ValueError("E cannot be larger than the number of possible values")
    r = rng if rng is not None else _random
    sel = r.sample(possible[:-1], E - 1)
    return np.sort(np.array(sel + [M], dtype=np.int64)).astype(np.int32)


def routing_table(offs, M: int, block_m: int):
    """Routing buffer ``[hist E | start E | total 1 | map grid_m_ub]`` (int32).

    kernels/forward.py:296-365 (``_expt_data_kernel`` / ``_build_expt_data``):
    hist[e] = offs[e]-offs[e-1], start[e] = offs[e-1], blocks_e = cdiv(hist, BM),
    total = sum(blocks_e), map[pid] = (pid-cum_e) << 16 | e for
    cum_e <= pid < cum_e+blocks_e, else -1; grid_m_ub = cdiv(M, BM) + max(E-1, 0).
    """
    offs = [int(v) for v in np.asarray(offs).reshape(-1)]
    E = len(offs)
    grid_m_ub = -(-M // block_m) + max(E - 1, 0)
    hist, start, mp = [], [], []
    prev, cum = 0, 0
    owners = {}
    for e, off in enumerate(offs):
        h = off - prev
        hist.append(h)
        start.append(prev)
        nb = -(-h // block_m) if h > 0 else 0
        for b in range(nb):
            owners[cum + b] = (b << 16) | e
        cum += nb
        prev = off
    for pid in range(grid_m_ub):
        mp.append(owners.get(pid, -1))
    return np.array(hist + start + [cum] + mp, dtype=np.int64).astype(np.int32), grid_m_ub


def xcd_swizzle(pid: int, domain: int, X: int) -> int:
    """kernels/forward.py:31-36: give each of X XCDs a contiguous logical range."""
    per = domain // X
    extra = domain % X
    g = pid % X
    return g * per + min(g, extra) + pid // X


def pid_grid(pid: int, num_m: int, num_n: int, group_m: int):
    """kernels/forward.py:38-51: GROUP_M band ordering, column-major within a band."""
    if group_m == 1:
        return pid // num_n, pid % num_n
    in_group = group_m * num_n
    gid = pid // in_group
    first = gid * group_m
    size = min(num_m - first, group_m)
    return first + (pid % size), (pid % in_group) // size


def tile_schedule(offs, M: int, N: int, block_m: int, block_n: int, group_m: int, xcd: int):
    """pid -> (pid_m, pid_n) or (-1, -1) for padding pids (kernels/forward.py:111-127).

    Grid = (cdiv(M,BM)+E-1) * cdiv(N,BN); pids >= total_tiles*grid_n exit.
    """
    buf, grid_m_ub = routing_table(offs, M, block_m)
    E = len(np.asarray(offs).reshape(-1))
    total = int(buf[2 * E])
    grid_n = -(-N // block_n)
    dom = total * grid_n
    out = []
    for pid in range(grid_m_ub * grid_n):
        if pid >= dom:
            out.append((-1, -1))
            continue
        t = xcd_swizzle(pid, dom, xcd) if xcd != 1 else pid
        out.append(pid_grid(t, total, grid_n, group_m))
    return np.array(out, dtype=np.int32).reshape(-1, 2)


def band_tile(blocks: int, grid_n: int, group_m: int, local: int):
    """(m-block, column tile) of tile ``local`` of one group in the build's
    expert-aligned band order.

    Not the reference's order: kernels/forward.py:38-51 cuts GROUP_M bands
    from the global m-block index, so a band can span two experts.  The build
    keeps each group's ``blocks x grid_n`` tiles contiguous and cuts the
    group's m-blocks into ``cdiv(blocks, group_m)`` balanced bands (height
    ``cdiv(blocks, nbands)``, the last band shorter), column-major inside a
    band.
    """
    g = max(int(group_m), 1)
    nbands = -(-blocks // g)
    bh = -(-blocks // nbands)
    b = min(local // (bh * grid_n), nbands - 1)
    in_band = local - b * bh * grid_n
    hb = blocks - b * bh if b == nbands - 1 else bh
    col = in_band // hb
    return b * bh + (in_band - col * hb), col


def fwd_tile_order(offs, M: int, N: int, block_m: int, block_n: int, group_m: int, xcd: int) -> np.ndarray:
    """The build's forward tile order: program id -> ``(expert, row0, rows,
    n0, cols)``, or five -1s for programs that compute nothing.

    Grid = ``(cdiv(M, BM) + E - 1) * cdiv(N, BN)`` programs, as the
    reference's (kernels/forward.py:347, 111-127).  A program id below the
    tile count is mapped by the XCD swizzle (kernels/forward.py:31-36) over
    the tile domain, then to the group whose tiles hold that index (groups in
    order, each group's tiles contiguous) and through ``band_tile``.  A tile
    holds rows ``row0 = offs[e-1] + block*BM`` up to the group's end, BM at
    most, and none at or past M.
    """
    offs = [int(v) for v in np.asarray(offs).reshape(-1)]
    E = len(offs)
    groups = []
    prev = 0
    for off in offs:
        h = off - prev
        groups.append((prev, h, -(-h // block_m) if h > 0 else 0))
        prev = off
    grid_n = -(-N // block_n)
    tiles = sum(nb for _, _, nb in groups) * grid_n
    programs = (-(-M // block_m) + max(E - 1, 0)) * grid_n
    out = np.full((programs, 5), -1, dtype=np.int64)
    for pid in range(min(programs, tiles)):
        t = xcd_swizzle(pid, tiles, xcd) if xcd > 1 else pid
        base = 0
        for e, (start, h, nb) in enumerate(groups):
            if nb and base <= t < base + nb * grid_n:
                block, col = band_tile(nb, grid_n, group_m, t - base)
                row0 = start + block * block_m
                rows = min(M - row0, h - block * block_m, block_m)
                if rows > 0:
                    out[pid] = (e, row0, rows, col * block_n, min(N - col * block_n, block_n))
                break
            base += nb * grid_n
    return out


# ----------------------------------------------------------------------------
# grouped GEMMs (dequantize -> per-group matmul)
# ----------------------------------------------------------------------------


def _bounds(offs):
    offs = [int(v) for v in np.asarray(offs).reshape(-1)]
    prev = 0
    for g, off in enumerate(offs):
        yield g, prev, off
        prev = off


def grouped_mm(a_q, a_s, b_q, b_s, offs, a_elem="e4m3", b_elem="e4m3", dtype=np.float64):
    """out[s:e] = A[s:e] @ B[g]^T per group, from dequantized operands.

    kernels/forward.py:461-606 (``triton_mxfp8_grouped_mm``) / forward.py:81-294:
    A (M,K) + scales (M,K/32); B (E,N,K) + scales (E,N,K/32); groups are
    cumulative end offsets, group g = rows [offs[g-1], offs[g]).  Rows past
    offs[-1] are not written by the reference (left uninitialised); here they
    are NaN so a test can never compare them by accident.  Returns float
    (``dtype``) before the bf16 store.
    """
    A = dequant(a_q, a_s, a_elem, dtype=dtype)
    B = dequant(b_q, b_s, b_elem, dtype=dtype)
    M = A.shape[0]
    N = B.shape[1]
    out = np.full((M, N), np.nan, dtype=dtype)
    for g, s, e in _bounds(offs):
        if e > s:
            out[s:e] = A[s:e] @ B[g].T
    return out


def wgrad(go_t_q, go_s, ia_t_q, ia_s, offs, dtype=np.float64):
    """out[g] = go_t[:, s:e] @ ia_t[:, s:e]^T, shape (E, N, K).

    kernels/backward.py:31-104 and 217-305 (``triton_mxfp8_wgrad``): go_t (N,M)
    and ia_t (K,M) quantized along M with per-32-token scales (N,M/32), (K,M/32);
    an empty group gives zeros.  The reference stores ``acc.to(bf16)`` whatever
    ``out_dtype`` is (backward.py:103, 214); callers round with
    ``f32_to_bf16_bits``.
    """
    GO = dequant(go_t_q, go_s, dtype=dtype)
    IA = dequant(ia_t_q, ia_s, dtype=dtype)
    offs = np.asarray(offs).reshape(-1)
    out = np.zeros((len(offs), GO.shape[0], IA.shape[0]), dtype=dtype)
    for g, s, e in _bounds(offs):
        if e > s:
            out[g] = GO[:, s:e] @ IA[:, s:e].T
    return out


def grouped_mm_hp(a_f32, b_f32, offs, dtype=np.float64):
    """Unquantized per-group reference (torch._grouped_mm on bf16 inputs;
    test_correctness.py:48-50)."""
    M = a_f32.shape[0]
    out = np.full((M, b_f32.shape[1]), np.nan, dtype=dtype)
    for g, s, e in _bounds(offs):
        if e > s:
            out[s:e] = a_f32[s:e].astype(dtype) @ b_f32[g].astype(dtype).T
    return out


# ----------------------------------------------------------------------------
# error metrics
# ----------------------------------------------------------------------------


def sqnr_db(ref, approx) -> float:
    """test_correctness.py:20-23: 20*log10(||ref|| / ||ref - approx||)."""
    ref = np.asarray(ref, dtype=np.float64)
    approx = np.asarray(approx, dtype=np.float64)
    ps = np.linalg.norm(ref.ravel())
    pn = np.linalg.norm((ref - approx).ravel())
    if pn == 0:
        return math.inf
    return 20.0 * math.log10(ps / pn)


def rel_fro(ref, approx) -> float:
    """||approx - ref||_F / ||ref||_F."""
    ref = np.asarray(ref, dtype=np.float64)
    approx = np.asarray(approx, dtype=np.float64)
    d = np.linalg.norm(ref.ravel())
    return float(np.linalg.norm((approx - ref).ravel()) / (d if d else 1.0))


PINNING = {
    "e4m3_from_f32": "torch's float8_e4m3fn cast on every bf16 pattern, their fp32 neighbours, "
                     "2**k-scaled copies and random fp32 (tests/test_oracle.py)",
    "e2m1_from_f32": "brute-force nearest-value search with ties to the even code over a dense grid",
    "mx_scales/to_mx": "closed-form KATs (amax at binade edges, zero/denormal/NaN/inf blocks) and the "
                       "FLOOR invariant amax*2**(127-s) in [256, 512) (e4m3) / [4, 8) (e2m1); "
                       "committed golden vectors tests/golden/",
    "dequant": "e4m3 table vs torch float8_e4m3fn->float32 for all 256 codes; e2m1 table vs OCP spec",
    "generate_jagged_offs": "invariants (sorted, distinct, multiples, last=M) and errors",
    "routing_table": "hand-derived KAT (E=4, offs=[96,352,640,1024], BM=128) plus brute force",
    "xcd_swizzle/pid_grid": "KAT (D=10, X=8) and bijection over many domains",
    "step_major": "hand KAT (3 rows x 5 blocks: word values and 127 padding); exact inverse "
                  "plain_from_step_major on random scales of many shapes",
    "band_tile/fwd_tile_order": "hand-derived KAT (E=4, offs=[96,352,640,1024], BM=BN=128, N=256, "
                                "GROUP_M=2); brute force: every output element of every group covered "
                                "by exactly one program, none past offs[-1]; equal to the reference's "
                                "routing map (routing_table) with one column tile and bands of one block",
    "grouped_mm/wgrad": "closed forms: E=1 equals a plain matmul; unit scales reduce to fp8 matmul; "
                        "zero inputs give zeros; SQNR vs the unquantized product",
}
