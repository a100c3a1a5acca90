"""mxgg_grouped_mm_noalloc, the allocation-free variant of mxgg_grouped_mm
(its workspace is a device array inside libmxgg), called through the C ABI:
bit-identical to mxgg_grouped_mm given a workspace of the same size, on two
calls in a row (the second smaller, so it runs on what the first left in the
array), and within the oracle's tolerance.  (The rejection of calls too large
for the array is a host check, tested on the CPU in test_boundary.py.)"""

import numpy as np
import pytest
import torch

from helpers import bits_u8, seeded_offs
from oracle import mx_oracle as O

pytestmark = pytest.mark.gpu


def _operands(E, M, N, K, seed, dev):
    import kernels
    g = torch.Generator(device=dev).manual_seed(seed)
    a = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    b = (torch.randn((E, N, K), device=dev, generator=g) * 0.02).to(torch.bfloat16)
    sa, qa = kernels.to_mx(a)
    sb, qb = kernels.to_mx(b)
    return qa.view(torch.uint8), sa, qb.view(torch.uint8), sb


def _args(qa, sa, qb, sb, offs, out, E, M, N, K):
    from kernels import _lib
    return (qa.data_ptr(), qa.stride(0), sa.data_ptr(), sa.stride(0),
            qb.data_ptr(), _lib.FMT_E4M3, qb.stride(1), qb.stride(0),
            sb.data_ptr(), sb.stride(1), sb.stride(0),
            offs.data_ptr(), E, M, N, K,
            out.data_ptr(), _lib.DTYPE_BF16, out.stride(0), 0, 0, 0, 0)


def test_noalloc_matches_workspace_entry_point(gpu):
    from kernels import _lib
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    ws = torch.empty(_lib.NOALLOC_SCRATCH_BYTES, dtype=torch.uint8, device=gpu)
    # first call: a sweep shape whose last round is split (partial tiles in the
    # array after the scales); second: smaller, with ragged and empty groups
    for E, M, N, K, offs in ((1, 16640, 2048, 8192, np.array([16000], np.int32)),
                             (8, 16640, 2048, 5120, seeded_offs(8, 16640, seed=5)),
                             (4, 1000, 384, 256, np.array([0, 300, 300, 992], np.int32))):
        print(f"noalloc E={E} M={M} N={N} K={K} offs={list(offs)}", flush=True)
        qa, sa, qb, sb = _operands(E, M, N, K, seed=E + K, dev=gpu)
        offs_t = torch.tensor(offs, dtype=torch.int32, device=gpu)
        want = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        got = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=gpu)
        _lib.check(lib.mxgg_grouped_mm(*_args(qa, sa, qb, sb, offs_t, want, E, M, N, K),
                                       ws.data_ptr(), ws.numel(), stream))
        _lib.check(lib.mxgg_grouped_mm_noalloc(*_args(qa, sa, qb, sb, offs_t, got, E, M, N, K), stream))
        torch.cuda.synchronize()
        rows = int(offs[-1])
        assert torch.equal(got[:rows].view(torch.int16), want[:rows].view(torch.int16))
        assert torch.isnan(got[rows:].float()).all()           # rows past offs[-1] untouched
        # and against the oracle on a slice of rows across a group boundary
        r0 = max(0, int(offs[0]) - 64)
        so = np.clip(np.asarray(offs, np.int64) - r0, 0, 128)
        ref = O.grouped_mm(bits_u8(qa[r0:r0 + 128]), bits_u8(sa[r0:r0 + 128]), bits_u8(qb[:, :128]),
                           bits_u8(sb[:, :128]), so)
        n = int(min(128, rows - r0))
        assert O.rel_fro(ref[:n], got[r0:r0 + n, :128].float().cpu().numpy()) <= 3e-3
