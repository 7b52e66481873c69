"""Static check of the kernels' gfx950 assembly for the vector-memory store-data hazard.

A store of more than 64 bits (buffer_store_dwordx4 / global_store_dwordx4) reads its data
registers after it issues, and an instruction that overwrites one of them needs at least
one wait state after the store.  The compiler once left none, where a store ended a loop
body and the loop header's first instruction reused the registers; the first dword of some
lanes was then stored wrong, differently from run to run.  The kernels now follow every
16-byte store with a statement that reads the stored registers and waits two wait states.
This test compiles each kernel source to device assembly with the library's own flags and
requires two wait states (instructions, or s_nop N counting N + 1) between every 16-byte
store and the next write of any of its data registers, falling through block labels."""
import re
import subprocess
from pathlib import Path

import pytest

from my_own_cnn_amd import build as B

KERNEL_SOURCES = ["qconv_igemm.hip", "qconv_stem.hip", "qconv_band.hip", "qconv_stream.hip", "qconv_direct.hip",
                  "gemm_i32.hip", "conv_f32.hip", "qconv_qi32.hip", "qconv_dot4.hip",
                  "qconv_qi32_band.hip", "qconv_qi32_route.hip", "qconv_flat.hip", "qconv_pipe.hip"]


def _regs(spec):
    m = re.match(r"([va])\[(\d+):(\d+)\]", spec)
    if m:
        return {(m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", spec)
    return {(m.group(1), int(m.group(2)))} if m else set()


def store_gaps(asm_lines):
    """(function, store, first overwrite, wait states) for every 16-byte store."""
    out = []
    func = None
    lines = [ln.strip() for ln in asm_lines]
    for i, t in enumerate(lines):
        m = re.match(r"^(_Z\S+):", t)
        if m:
            func = m.group(1)
            continue
        if not (t.startswith("buffer_store_dwordx4") or t.startswith("global_store_dwordx4")):
            continue
        ops = [o.strip() for o in t.split(None, 1)[1].split(",")]
        data = _regs(ops[1] if t.startswith("global_store") else ops[0])  # global: vaddr, vdata
        waits = 0
        for u in lines[i + 1:i + 40]:
            if not u or u.startswith(";") or u.startswith("."):
                continue  # comments, directives and block labels: fall through
            if u.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")) or u.startswith("_Z"):
                break
            nop = re.match(r"s_nop (\d+)", u)
            if nop:
                waits += int(nop.group(1)) + 1
                continue
            parts = u.split(None, 1)
            writes = (len(parts) > 1 and not parts[0].startswith(("buffer_store", "global_store", "ds_write", "s_")))
            if writes and _regs(parts[1].split(",")[0].strip()) & data:
                out.append((func, t, u, waits))
                break
            waits += 1
    return out


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory):
    cc = B.hipcc()
    outdir = tmp_path_factory.mktemp("isa")
    procs = {}
    for src in KERNEL_SOURCES:
        dst = outdir / (src + ".s")
        cmd = [cc, *B.common_flags(), "--cuda-device-only", "-S", str(B.CSRC / src), "-o", str(dst)]
        procs[src] = (subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), dst)
    asm = {}
    for src, (p, dst) in procs.items():
        log, _ = p.communicate(timeout=600)
        assert p.returncode == 0, log
        asm[src] = Path(dst).read_text().splitlines()
    return asm


@pytest.mark.parametrize("src", KERNEL_SOURCES)
def test_every_wide_store_keeps_its_data_two_wait_states(kernel_asm, src):
    gaps = store_gaps(kernel_asm[src])
    short = [g for g in gaps if g[3] < 2]
    assert not short, "\n".join(f"{f}: {s} -> {u} after {w} wait states" for f, s, u, w in short[:10])


def test_the_check_finds_a_missing_gap():
    # the pattern of the original failure, and the fixed form
    bad = ["_Zkern:", "buffer_store_dwordx4 v[160:163], v203, s[4:7], s26 offen nt", ".LBB0_130:",
           "v_add_u32_e32 v160, s24, v195"]
    good = ["_Zkern:", "buffer_store_dwordx4 v[160:163], v203, s[4:7], s26 offen nt", "s_nop 1",
            ".LBB0_130:", "v_add_u32_e32 v160, s24, v195"]
    addr_only = ["_Zkern:", "global_store_dwordx4 v[0:1], a[0:3], off", "v_accvgpr_read_b32 v0, a0"]
    assert [g[3] for g in store_gaps(bad)] == [0]
    assert [g[3] for g in store_gaps(good)] == [2]
    assert store_gaps(addr_only) == []  # v[0:1] is the address, a[0:3] the data
