"""CPU tests that pin the oracle (oracle/mx_oracle.py) before it is trusted.

Each check is independent of the oracle's own formulas: torch's float8 cast
(the routine the reference's ``to_mx`` calls, utils.py:102), brute-force
nearest-value searches, hand-derived known answers, closed-form identities
and invariants.  A plausible mistake in the oracle (wrong rounding, an
off-by-one exponent, a transposed operand, a dropped group) fails one of them.
"""

import random

import numpy as np
import pytest
import torch

from oracle import mx_oracle as O

# ---------------------------------------------------------------- e4m3 cast


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.float8_e4m3fn) \
        .view(torch.uint8).numpy()


def test_e4m3_every_bf16_pattern_matches_torch():
    f = O.bf16_bits_to_f32(np.arange(65536, dtype=np.uint16))
    np.testing.assert_array_equal(O.e4m3_from_f32(f), _torch_e4m3(f))


def test_e4m3_fp32_neighbours_and_scaled_copies_match_torch():
    f = O.bf16_bits_to_f32(np.arange(65536, dtype=np.uint16))
    f = f[np.isfinite(f)]
    up = np.nextafter(f, np.float32(np.inf))
    dn = np.nextafter(f, np.float32(-np.inf))
    xs = [up, dn]
    for k in (-3, -1, 1, 3):
        xs.append((f * np.float32(2.0 ** k)).astype(np.float32))
    x = np.concatenate(xs).astype(np.float32)
    np.testing.assert_array_equal(O.e4m3_from_f32(x), _torch_e4m3(x))


def test_e4m3_random_fp32_matches_torch():
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    np.testing.assert_array_equal(O.e4m3_from_f32(x), _torch_e4m3(x))


def test_e4m3_decode_table_matches_torch():
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    same = (t == O.E4M3_TABLE) | (np.isnan(t) & np.isnan(O.E4M3_TABLE))
    assert same.all()


def test_e4m3_round_trip_of_every_code():
    codes = np.arange(256, dtype=np.uint8)
    vals = O.E4M3_TABLE[codes]
    ok = ~np.isnan(vals)
    np.testing.assert_array_equal(O.e4m3_from_f32(vals[ok]), codes[ok])


# ---------------------------------------------------------------- e2m1 cast


def _e2m1_brute(x: np.ndarray) -> np.ndarray:
    """Nearest representable e2m1 magnitude, ties to the even mantissa bit,
    saturating at 6; NaN -> max magnitude.  Pure search, no bit arithmetic."""
    mags = O.E2M1_TABLE[:8].astype(np.float64)
    out = np.empty(x.shape, dtype=np.uint8)
    for i, v in enumerate(x.astype(np.float64)):
        sign = 8 if np.signbit(v) else 0
        if np.isnan(v):
            out[i] = 7 | sign
            continue
        a = min(abs(v), 6.0)
        d = np.abs(mags - a)
        best = np.flatnonzero(d == d.min())
        if len(best) > 1:                   # tie: pick the code with mantissa bit 0
            best = [c for c in best if c % 2 == 0]
        c = int(best[0])
        out[i] = (c | sign) if c else (0 | sign)
    return out


def test_e2m1_matches_brute_force_on_dense_grid():
    grid = np.concatenate([np.linspace(-7, 7, 5601), np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0,
                                                               -0.25, -2.5, 6.0, 100.0, -1e30, np.inf,
                                                               -np.inf, np.nan, -0.0, 1e-40])])
    x = grid.astype(np.float32)
    np.testing.assert_array_equal(O.e2m1_from_f32(x), _e2m1_brute(x))


def test_e2m1_pack_order_matches_torch_x2_convention():
    # Float4_e2m1fn_x2: val0 in bits 3..0, val1 in bits 7..4
    n = np.array([[1, 2, 3, 4]], dtype=np.uint8)
    np.testing.assert_array_equal(O.pack_e2m1(n), np.array([[0x21, 0x43]], dtype=np.uint8))
    np.testing.assert_array_equal(O.unpack_e2m1(O.pack_e2m1(n)), n)


# ---------------------------------------------------------------- to_mx (FLOOR)


def _block(values, fill=0.0):
    b = np.full(32, fill, dtype=np.float32)
    b[: len(values)] = values
    return b


@pytest.mark.parametrize("amax,scale", [
    (1.0, 119),                # floor(log2 1) = 0 -> 0 - 8 + 127
    (448.0, 127),              # floor(log2 448) = 8
    (511.99, 127),
    (512.0, 128),
    (2.0 ** -118, 1),
    (2.0 ** -119, 0),          # clamps at 0
    (2.0 ** -126, 0),
    (2.0 ** -140, 0),          # denormal amax -> fp32 tiny -> 0
    (3.0e38, 246),             # exponent field 254
])
def test_to_mx_scale_kats(amax, scale):
    s, _ = O.to_mx(_block([amax, -amax / 3]), src="f32")
    assert int(s[0]) == scale


def test_to_mx_special_blocks():
    z, q = O.to_mx(np.zeros(32, np.float32), src="f32")
    assert z[0] == 0 and (q == 0).all()
    s, q = O.to_mx(_block([np.nan, 1.0]), src="f32")
    assert s[0] == 247 and q[0] == 0x7F and q[1] == 0          # 1.0 * 2**-120 -> 0
    s, q = O.to_mx(_block([-np.inf, 7.0]), src="f32")
    assert s[0] == 247 and q[0] == 0xFE                        # -inf clamps to -448
    s, q = O.to_mx(_block([-0.0, 1.0]), src="f32")
    assert q[0] == 0x80                                        # negative zero kept
    # denormal-only block: scale 0 multiplies by 2**127, values become normal e4m3
    s, q = O.to_mx(_block([2.0 ** -130]), src="f32")
    assert s[0] == 0 and O.E4M3_TABLE[q[0]] == 2.0 ** -3


def test_to_mx_floor_invariant_random():
    """For finite, non-tiny blocks amax * 2**(127-s) lies in [256, 512)
    (e4m3, max_pow2 8) resp. [4, 8) (e2m1, max_pow2 2)."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((400, 256)) * np.exp(rng.uniform(-20, 20, (400, 1)))).astype(np.float32)
    for elem, lo in (("e4m3", 256.0), ("e2m1", 4.0)):
        s, _ = O.to_mx(x, src="f32", elem=elem)
        amax = np.abs(x.reshape(400, 8, 32)).max(-1).astype(np.float64)
        r = amax * np.exp2(127.0 - s.astype(np.float64))
        assert ((r >= lo) & (r < 2 * lo)).all()


def test_to_mx_dequant_error_bound():
    """|dequant(q) - x| <= half an e4m3 ulp of the scaled value, or saturation."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 128)).astype(np.float32)
    s, q = O.to_mx(x, src="f32")
    d = O.dequant(q, s)
    scaled_err = np.abs(d - x) * np.exp2(127.0 - np.repeat(s, 32, axis=1).astype(np.float64))
    xs = np.abs(x) * np.exp2(127.0 - np.repeat(s, 32, axis=1).astype(np.float64))
    ulp = np.exp2(np.floor(np.log2(np.maximum(xs, 2.0 ** -6))) - 3)
    assert ((scaled_err <= ulp / 2 + 1e-12) | (xs >= 448.0)).all()


def test_to_mx_bf16_path_matches_f32_path():
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((32, 64)).astype(np.float32)).to(torch.bfloat16)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    s1, q1 = O.to_mx(bits, src="bf16")
    s2, q2 = O.to_mx(x.float().numpy(), src="f32")
    np.testing.assert_array_equal(s1, s2)
    np.testing.assert_array_equal(q1, q2)


def test_to_mx_asserts_block_divisibility():
    with pytest.raises(AssertionError):
        O.to_mx(np.zeros((2, 48), np.float32), src="f32")


def test_golden_cfg1_replays():
    """The committed fixture still equals what the oracle produces."""
    import os
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1.npz"))
    s, q = O.to_mx(z["a_bf16"], src="bf16")
    np.testing.assert_array_equal(s, z["a_scales"])
    np.testing.assert_array_equal(q, z["a_q"])
    s, q = O.to_mx(z["b_bf16"], src="bf16")
    np.testing.assert_array_equal(s, z["b_scales"])
    np.testing.assert_array_equal(q, z["b_q"])
    out = O.grouped_mm(z["a_q"], z["a_scales"], z["b_q"], z["b_scales"], z["offs"])
    np.testing.assert_array_equal(O.f32_to_bf16_bits(out.astype(np.float32)), z["out_bf16"])
    assert z["offs"][-1] == 1024 and (z["offs"] % 32 == 0).all()


# ---------------------------------------------------------------- bf16 rounding


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(4)
    x = rng.integers(0, 2 ** 32, size=500_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[~np.isnan(x)]
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(x), ref)


# ---------------------------------------------------------------- offsets


def test_generate_jagged_offs_invariants_and_errors():
    for E in (1, 2, 4, 8, 64):
        o = O.generate_jagged_offs(E, 16640, 32, rng=random.Random(E))
        assert len(o) == E and o[-1] == 16640 and (np.diff(o) > 0).all() and (o % 32 == 0).all()
    with pytest.raises(ValueError):
        O.generate_jagged_offs(2, 100, 32)
    with pytest.raises(ValueError):
        O.generate_jagged_offs(5, 128, 32)


def test_generate_jagged_offs_follows_random_sample():
    """Same RNG consumption as utils.py:47: one random.sample call."""
    r1, r2 = random.Random(123), random.Random(123)
    o = O.generate_jagged_offs(8, 16640, 32, rng=r1)
    want = sorted(r2.sample(list(range(32, 16640, 32)), 7)) + [16640]
    assert o.tolist() == want


# ---------------------------------------------------------------- routing / schedule


def test_routing_table_kat():
    buf, ub = O.routing_table([96, 352, 640, 1024], 1024, 128)
    assert ub == 11
    assert buf.tolist() == [96, 256, 288, 384, 0, 96, 352, 640, 9,
                            0x0, 0x1, 0x10001, 0x2, 0x10002, 0x20002, 0x3, 0x10003, 0x20003, -1, -1]


def test_routing_table_brute_force():
    rng = random.Random(5)
    for _ in range(50):
        E = rng.randint(1, 9)
        M = rng.randint(1, 40) * 32
        BM = rng.choice((32, 64, 128, 256))
        cuts = sorted(rng.randint(0, M) for _ in range(E - 1)) + [M]
        buf, ub = O.routing_table(cuts, M, BM)
        # brute force: enumerate tiles group by group
        tiles, prev = [], 0
        for e, c in enumerate(cuts):
            for b in range(-(-(c - prev) // BM) if c > prev else 0):
                tiles.append((b << 16) | e)
            prev = c
        assert buf[2 * E] == len(tiles)
        assert buf[2 * E + 1:].tolist() == tiles + [-1] * (ub - len(tiles))
        # every row of every group is covered exactly once
        cover = np.zeros(M, int)
        starts = buf[E:2 * E]
        for t in tiles:
            e, b = t & 0xFFFF, t >> 16
            lo = starts[e] + b * BM
            cover[lo:min(lo + BM, cuts[e])] += 1
        assert (cover[: cuts[-1]] == 1).all()


def test_xcd_swizzle_kat_and_bijection():
    assert [O.xcd_swizzle(p, 10, 8) for p in range(10)] == [0, 2, 4, 5, 6, 7, 8, 9, 1, 3]
    for D in (1, 7, 8, 9, 63, 64, 65, 520, 1040, 2081):
        for X in (1, 2, 4, 8):
            assert sorted(O.xcd_swizzle(p, D, X) for p in range(D)) == list(range(D))
    # each XCD (pid % X) owns a contiguous logical range
    D, X = 100, 8
    for g in range(X):
        vals = sorted(O.xcd_swizzle(p, D, X) for p in range(g, D, X))
        assert vals == list(range(vals[0], vals[0] + len(vals)))


def test_pid_grid_bijection_and_band_order():
    for nm, nn, gm in ((65, 8, 8), (7, 3, 4), (1, 5, 8), (130, 16, 16), (9, 9, 1)):
        seen = {O.pid_grid(p, nm, nn, gm) for p in range(nm * nn)}
        assert seen == {(m, n) for m in range(nm) for n in range(nn)}
    # column-major inside a band of GROUP_M m-tiles
    assert [O.pid_grid(p, 8, 4, 4) for p in range(6)] == [(0, 0), (1, 0), (2, 0), (3, 0), (0, 1), (1, 1)]


def test_tile_schedule_covers_every_tile_once():
    offs = [100, 612, 612, 2000]
    sched = O.tile_schedule(offs, 2000, 700, 128, 128, 8, 8)
    live = sched[sched[:, 0] >= 0]
    buf, _ = O.routing_table(offs, 2000, 128)
    total = int(buf[2 * 4])
    assert len(live) == total * 6
    assert len({tuple(r) for r in live.tolist()}) == len(live)


def test_fwd_tile_order_kat():
    """Hand-derived from the band rule: groups of 1, 2, 3, 3 m-blocks of 128
    rows, 2 column tiles, GROUP_M 2, no XCD swizzle.  Group 2 (3 blocks) gets
    2 bands (heights 2 and 1), column-major inside each."""
    offs = [96, 352, 640, 1024]
    got = O.fwd_tile_order(offs, 1024, 256, 128, 128, 2, 1)
    ebc = [(0, 0, 0), (0, 0, 1),
           (1, 0, 0), (1, 1, 0), (1, 0, 1), (1, 1, 1),
           (2, 0, 0), (2, 1, 0), (2, 0, 1), (2, 1, 1), (2, 2, 0), (2, 2, 1),
           (3, 0, 0), (3, 1, 0), (3, 0, 1), (3, 1, 1), (3, 2, 0), (3, 2, 1)]
    start = {0: 0, 1: 96, 2: 352, 3: 640}
    rows = {(0, 0): 96, (1, 0): 128, (1, 1): 128, (2, 0): 128, (2, 1): 128, (2, 2): 32,
            (3, 0): 128, (3, 1): 128, (3, 2): 128}
    want = [(e, start[e] + 128 * b, rows[(e, b)], 128 * c, 128) for e, b, c in ebc]
    assert got.shape == ((8 + 3) * 2, 5)
    assert [tuple(r) for r in got[:18].tolist()] == want
    assert (got[18:] == -1).all()
    # the XCD swizzle (D=18, X=8) permutes the same tiles
    sw = O.fwd_tile_order(offs, 1024, 256, 128, 128, 2, 8)
    assert [tuple(r) for r in sw[:3].tolist()] == [want[0], want[3], want[6]]
    assert sorted(tuple(r) for r in sw[:18].tolist()) == sorted(want)


@pytest.mark.parametrize("seed", range(6))
def test_fwd_tile_order_covers_each_output_once(seed):
    """Brute force: every (row, column) of every group is computed by exactly
    one program, and nothing at or past offs[-1]; empty groups, more than 64
    groups, both tile sizes, several GROUP_M and XCD widths."""
    rng = np.random.default_rng(seed)
    E = int(rng.choice([1, 3, 8, 80]))
    sizes = rng.integers(0, 5, size=E) * int(rng.choice([32, 96, 7]))
    if E > 4:
        sizes[rng.choice(E, E // 5, replace=False)] = 0
    offs = np.cumsum(sizes).astype(np.int64)
    M = int(offs[-1]) + int(rng.integers(0, 300))
    N = int(rng.choice([96, 256, 700]))
    for BM in (128, 256):
        for gm in (1, 3, 12):
            for xcd in (1, 8):
                got = O.fwd_tile_order(offs, M, N, BM, BM, gm, xcd)
                cover = np.zeros((M, N), np.int32)
                for e, r0, rows, n0, cols in got.tolist():
                    if e < 0:
                        continue
                    lo = offs[e - 1] if e else 0
                    assert lo <= r0 and r0 + rows <= offs[e] and rows > 0 and 0 < cols <= BM
                    cover[r0:r0 + rows, n0:n0 + cols] += 1
                assert (cover[: int(offs[-1])] == 1).all() and (cover[int(offs[-1]):] == 0).all()


def test_fwd_tile_order_reduces_to_reference_map():
    """With one column tile, bands of one m-block and no swizzle, the build's
    order is the reference's m-block order (kernels/forward.py:320-338)."""
    for E, M, BM, seed in ((4, 1024, 128, 1), (8, 16640, 256, 2), (70, 4096, 128, 3)):
        offs = O.generate_jagged_offs(E, M, 32, rng=random.Random(seed))
        buf, gub = O.routing_table(offs, M, BM)
        got = O.fwd_tile_order(offs, M, 64, BM, 64, 1, 1)
        starts = [0] + [int(v) for v in offs[:-1]]
        for pid, code in enumerate(buf[2 * E + 1:].tolist()):
            if code < 0:
                assert got[pid, 0] == -1
            else:
                e, b = code & 0xFFFF, code >> 16
                assert (got[pid, 0], got[pid, 1]) == (e, starts[e] + b * BM)


def test_step_major_kat_and_inverse():
    s = np.arange(15, dtype=np.uint8).reshape(3, 5) + 100      # rows 0..2, blocks 0..4
    w = O.step_major(s)
    assert w.shape == (2, 3) and w.dtype == np.uint32
    # row 1: blocks 105..109 -> word 0 = 105 | 106<<8 | 107<<16 | 108<<24, word 1 = 109 | 127 127 127
    assert int(w[0, 1]) == 105 | 106 << 8 | 107 << 16 | 108 << 24
    assert int(w[1, 1]) == 109 | 127 << 8 | 127 << 16 | 127 << 24
    rng = np.random.default_rng(3)
    for shape in ((1, 4), (7, 8), (2, 5, 13), (3, 64, 520)):
        x = rng.integers(0, 255, size=shape, dtype=np.uint8)
        ws = O.step_major(x)
        assert ws.shape == shape[:-2] + (-(-shape[-1] // 4), shape[-2])
        np.testing.assert_array_equal(O.plain_from_step_major(ws, shape[-1]), x)


# ---------------------------------------------------------------- grouped GEMMs


def test_grouped_mm_e1_is_plain_matmul():
    rng = np.random.default_rng(6)
    a = rng.standard_normal((96, 64)).astype(np.float32)
    b = rng.standard_normal((1, 48, 64)).astype(np.float32)
    sa, qa = O.to_mx(a, src="f32")
    sb, qb = O.to_mx(b, src="f32")
    out = O.grouped_mm(qa, sa, qb, sb, [96])
    np.testing.assert_allclose(out, O.dequant(qa, sa) @ O.dequant(qb, sb)[0].T, rtol=0, atol=0)


def test_grouped_mm_unit_scales_reduce_to_fp8_matmul():
    rng = np.random.default_rng(7)
    qa = rng.integers(0, 0x7E, (64, 64), dtype=np.uint8)
    qb = rng.integers(0, 0x7E, (2, 32, 64), dtype=np.uint8)
    sa = np.full((64, 2), 127, np.uint8)
    sb = np.full((2, 32, 2), 127, np.uint8)
    out = O.grouped_mm(qa, sa, qb, sb, [40, 64])
    A = O.E4M3_TABLE[qa].astype(np.float64)
    B = O.E4M3_TABLE[qb].astype(np.float64)
    np.testing.assert_array_equal(out[:40], A[:40] @ B[0].T)
    np.testing.assert_array_equal(out[40:], A[40:] @ B[1].T)


def test_grouped_mm_scale_exponents_factor_out():
    """Raising one scale byte by k multiplies exactly that block's contribution by 2**k."""
    rng = np.random.default_rng(8)
    a = rng.standard_normal((8, 64)).astype(np.float32)
    b = rng.standard_normal((1, 4, 64)).astype(np.float32)
    sa, qa = O.to_mx(a, src="f32")
    sb, qb = O.to_mx(b, src="f32")
    base = O.grouped_mm(qa, sa, qb, sb, [8])
    sa2 = sa.copy()
    sa2[:, 1] += 3
    got = O.grouped_mm(qa, sa2, qb, sb, [8])
    A = O.dequant(qa, sa)
    B = O.dequant(qb, sb)[0]
    blk = A[:, 32:] @ B[:, 32:].T
    np.testing.assert_allclose(got, base + 7 * blk, rtol=1e-12, atol=1e-12)


def test_grouped_mm_group_boundaries_and_zero():
    rng = np.random.default_rng(9)
    qa = rng.integers(0, 0x7E, (64, 32), dtype=np.uint8)
    qb = np.zeros((3, 16, 32), np.uint8)
    sa = np.full((64, 1), 127, np.uint8)
    sb = np.full((3, 16, 1), 127, np.uint8)
    out = O.grouped_mm(qa, sa, qb, sb, [32, 32, 48])
    assert (out[:48] == 0).all() and np.isnan(out[48:]).all()   # rows past offs[-1] not written


def test_wgrad_matches_explicit_loop_and_empty_group():
    rng = np.random.default_rng(10)
    M, N, K = 128, 16, 8
    go = rng.standard_normal((M, N)).astype(np.float32)
    ia = rng.standard_normal((M, K)).astype(np.float32)
    sg, qg = O.to_mx(go.T.copy(), src="f32")
    si, qi = O.to_mx(ia.T.copy(), src="f32")
    offs = [32, 32, 128]
    out = O.wgrad(qg, sg, qi, si, offs)
    G = O.dequant(qg, sg).T
    I = O.dequant(qi, si).T
    ref = np.zeros((3, N, K))
    prev = 0
    for g, e in enumerate(offs):
        for m in range(prev, e):
            ref[g] += np.outer(G[m], I[m])
        prev = e
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)
    assert (out[1] == 0).all()


def test_quantized_gemm_sqnr_matches_reference_level():
    """The FLOOR recipe's SQNR vs the unquantized product is ~27.6 dB
    (README.md:33-34) -- a property of the format, checked on the oracle."""
    rng = np.random.default_rng(11)
    a = torch.from_numpy(rng.standard_normal((512, 512)).astype(np.float32)).to(torch.bfloat16)
    b = torch.from_numpy(rng.standard_normal((2, 256, 512)).astype(np.float32)).to(torch.bfloat16)
    ab = a.view(torch.int16).numpy().view(np.uint16)
    bb = b.view(torch.int16).numpy().view(np.uint16)
    sa, qa = O.to_mx(ab, src="bf16")
    sb, qb = O.to_mx(bb, src="bf16")
    offs = [192, 512]
    out = O.grouped_mm(qa, sa, qb, sb, offs)
    hp = O.grouped_mm_hp(O.bf16_bits_to_f32(ab), O.bf16_bits_to_f32(bb), offs)
    assert 27.0 <= O.sqnr_db(hp, out) <= 28.5


# ------------------------------------------- the torch CPU path (oracle/torch_ref.py)


def test_torch_ref_to_mx_matches_golden_and_oracle():
    """The torch restatement of to_mx (utils.py:84-105), which bench.py times on
    the host's cores, gives the golden fixture's bytes and scales, and the
    oracle's on special blocks (NaN, +-inf, zero, -0, denormal-only, saturating
    448 / 464 / 480 * 2**k)."""
    import os
    from oracle import torch_ref as T
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1.npz"))
    for name in ("a", "b"):
        x = torch.from_numpy(z[name + "_bf16"].view(np.int16)).view(torch.bfloat16)
        s, q = T.to_mx(x)
        np.testing.assert_array_equal(s.numpy(), z[name + "_scales"])
        np.testing.assert_array_equal(q.view(torch.uint8).numpy(), z[name + "_q"])
    vals = [np.nan, -np.inf, np.inf, 0.0, -0.0, 2.0 ** -130, 448.0 * 2 ** 5, 464.0 * 2 ** -3, 480.0, 1.0, -3.5]
    x = np.zeros((len(vals), 32), np.float32)
    rng = np.random.default_rng(12)
    for i, v in enumerate(vals):
        x[i] = rng.standard_normal(32).astype(np.float32) * (0.0 if v == 0.0 or v == 2.0 ** -130 else 0.5)
        x[i, 3] = v
    s, q = T.to_mx(torch.from_numpy(x))
    rs, rq = O.to_mx(x, src="f32")
    np.testing.assert_array_equal(s.numpy(), rs)
    np.testing.assert_array_equal(q.view(torch.uint8).numpy(), rq)


def test_torch_ref_grouped_mm_matches_golden():
    """Dequantize + one fp32 torch.matmul per group: within fp32 accumulation
    error of the fp64 oracle on BASELINE config 1 (golden fixture), every
    group (an empty one included) in place."""
    import os
    from oracle import torch_ref as T
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "cfg1.npz"))
    t = lambda a, dt=torch.uint8: torch.from_numpy(np.ascontiguousarray(a)).view(dt)
    out = T.grouped_mm(t(z["a_q"], torch.float8_e4m3fn), t(z["a_scales"]), t(z["b_q"], torch.float8_e4m3fn),
                       t(z["b_scales"]), z["offs"])
    ref = O.bf16_bits_to_f32(z["out_bf16"])
    got = out.float().numpy()
    assert O.rel_fro(ref, got) <= 4e-3          # bf16 rounding of both sides
    assert np.mean(O.f32_to_bf16_bits(got) == z["out_bf16"]) > 0.99
    # an empty group, rows past offs[-1] zero
    offs = [0, 512, 512, 1000]
    out = T.grouped_mm(t(z["a_q"], torch.float8_e4m3fn), t(z["a_scales"]), t(z["b_q"], torch.float8_e4m3fn),
                       t(z["b_scales"]), offs).float().numpy()
    ora = O.grouped_mm(z["a_q"], z["a_scales"], z["b_q"], z["b_scales"], offs)
    assert O.rel_fro(ora[:1000], out[:1000]) <= 4e-3 and (out[1000:] == 0).all()
