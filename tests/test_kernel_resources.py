"""Resource use of the built gfx950 kernels, read from the code objects that
the build embeds in ``libmxgg.so`` (no GPU needed).

The GEMM main loops hold 256 fp32 accumulators per lane next to two sets of
operand and scale registers; a register allocator that runs short spills to
per-lane scratch memory inside the loop, which costs several percent and has
happened before when one kernel carried several epilogues.  These checks fail
the CPU suite as soon as any kernel of the library uses scratch, spills, or
asks for more LDS than a CU holds.

Layout read here: a clang offload bundle (``__CLANG_OFFLOAD_BUNDLE__``, a
count, then per entry offset / size / target triple) per translation unit;
the gfx950 entry is an ELF code object whose NT_AMDGPU_METADATA note (type
32, owner "AMDGPU") holds msgpack kernel records.
"""

import os
import re
import struct

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "grouped-gemms_amd", "kernels", "libmxgg.so")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
LDS_BYTES_PER_CU = 160 * 1024


def _code_objects(blob: bytes, arch: str = "gfx950"):
    for m in re.finditer(re.escape(MAGIC), blob):
        base = m.start()
        (n,) = struct.unpack_from("<Q", blob, base + len(MAGIC))
        p = base + len(MAGIC) + 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", blob, p)
            p += 24
            triple = blob[p:p + tlen].decode()
            p += tlen
            if triple.endswith(arch) and size:
                yield blob[base + off: base + off + size]


def _metadata(elf: bytes):
    import msgpack
    assert elf[:4] == b"\x7fELF" and elf[4] == 2, "64-bit ELF code object expected"
    (shoff,) = struct.unpack_from("<Q", elf, 0x28)
    shentsize, shnum = struct.unpack_from("<HH", elf, 0x3A)
    for i in range(shnum):
        _, sh_type, _, _, off, size = struct.unpack_from("<IIQQQQ", elf, shoff + i * shentsize)
        if sh_type != 7:            # SHT_NOTE
            continue
        q = off
        while q < off + size:
            namesz, descsz, ntype = struct.unpack_from("<III", elf, q)
            q += 12
            owner = elf[q:q + namesz].rstrip(b"\0")
            q += (namesz + 3) & ~3
            desc = elf[q:q + descsz]
            q += (descsz + 3) & ~3
            if ntype == 32 and owner == b"AMDGPU":
                yield msgpack.unpackb(desc)


def _kernels():
    if not os.path.exists(LIB):
        pytest.skip("libmxgg.so is not built (run __graft_entry__.build())")
    blob = open(LIB, "rb").read()
    out = {}
    for co in _code_objects(blob):
        for md in _metadata(co):
            for k in md["amdhsa.kernels"]:
                out[k[".name"]] = k
    return out


def test_code_objects_found():
    ks = _kernels()
    names = " ".join(ks)
    for part in ("fwd_kernel", "wgrad_kernel", "fwd_quad_kernel", "fwd_reduce_kernel", "wgrad_reduce_kernel",
                 "scale_relayout_kernel", "quant_rows_kernel", "quant_tile_kernel", "schedule_kernel",
                 "routing_kernel"):
        assert part in names, f"no {part} in the gfx950 code objects"


def test_no_scratch_or_spills():
    bad = {n: (k[".private_segment_fixed_size"], k.get(".vgpr_spill_count", 0), k.get(".sgpr_spill_count", 0))
           for n, k in _kernels().items()
           if k[".private_segment_fixed_size"] or k.get(".vgpr_spill_count", 0) or k.get(".sgpr_spill_count", 0)}
    assert not bad, f"kernels using scratch (bytes/lane, VGPR spills, SGPR spills): {bad}"


def test_lds_fits_one_cu():
    for n, k in _kernels().items():
        assert k[".group_segment_fixed_size"] <= LDS_BYTES_PER_CU, n


def test_gemm_kernels_one_wave_per_simd():
    """The GEMM kernels are built for 4-wave workgroups (one wave per SIMD for
    256 x 256 tiles) with at most 512 registers per lane (``.vgpr_count`` is the unified count, AGPRs
    included); anything else means the tile configuration or launch bounds
    changed."""
    gemm = {n: k for n, k in _kernels().items() if re.search(r"(fwd|wgrad)_kernel", n)}
    assert gemm
    for n, k in gemm.items():
        assert k[".wavefront_size"] == 64, n
        assert k[".max_flat_workgroup_size"] == 256, n
        assert k.get(".agpr_count", 0) <= k[".vgpr_count"] <= 512, n
