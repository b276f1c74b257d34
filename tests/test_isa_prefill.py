"""Static check of the prefill kernels' gfx950 code (CPU only: hipcc -S).

Each wave stages its page of the next K/V tile with eight direct-to-LDS copies
(global_load_lds_dwordx4, issued from inline asm, which the compiler's wait
counting does not see).  If the compiler puts an ``s_waitcnt vmcnt`` between
those copies -- it did when a copy offset was built with v_mad_u64_u32 on a
register pair whose high half held a pending block-table load -- every tile
waits for its own copies and the kernel loses 10-15 %.  This test compiles
csrc/paged_prefill.hip with the library's flags and asserts that no basic
block of any instantiation has such a wait between its copies.
"""

import importlib.util
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "nano-vllm-practice_amd")


def _compile_to_asm(tmp_path):
    # the library's build script: same hipcc and flags
    spec = importlib.util.spec_from_file_location("femto_build", os.path.join(PKG, "build.py"))
    build = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(build)

    try:
        hipcc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path / "paged_prefill.s"
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    cmd = [hipcc, *flags, "--cuda-device-only", "-S", "-I", build.INCLUDE, "-I", build.CSRC,
           os.path.join(build.CSRC, "paged_prefill.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


def _kernels(asm):
    lines = asm.split("\n")
    starts = [(i, l.split(":")[0]) for i, l in enumerate(lines)
              if re.match(r"^_ZN5femto21attention_mfma_kernel\w+:", l)]
    for s, name in starts:
        e = next(j for j in range(s, len(lines)) if lines[j].startswith(".Lfunc_end"))
        yield name, lines[s:e]


def _blocks(body):
    block, name = [], "entry"
    for line in body:
        m = re.match(r"^(\.LBB[\w_]+):", line)
        if m:
            yield name, block
            block, name = [], m.group(1)
            continue
        t = line.strip()
        if t and not t.startswith((";", ".")):
            block.append(t)
    yield name, block


def test_no_wait_between_tile_copies(tmp_path):
    asm = _compile_to_asm(tmp_path)
    kernels = list(_kernels(asm))
    # {bf16, f16} x G {1, 2, 4} x {paged, paged with decode workers, dense} at head_dim 128, and
    # the paged ones again for head_dim < 128
    assert len(kernels) == 30
    bad, blocks_with_copies = [], 0
    for name, body in kernels:
        for bname, ins in _blocks(body):
            copies = [k for k, t in enumerate(ins) if t.startswith("global_load_lds_dwordx4")]
            if len(copies) < 2:
                continue
            blocks_with_copies += 1
            waits = [t for t in ins[copies[0]:copies[-1]] if t.startswith("s_waitcnt") and "vmcnt" in t]
            if waits:
                bad.append((name, bname, waits))
    assert blocks_with_copies >= 18
    assert not bad, f"vmcnt waits between direct-to-LDS copies: {bad[:4]}"


def test_copies_carry_hazard_wait_states(tmp_path):
    """Each direct-to-LDS copy is issued from inline asm, where the compiler
    inserts no hazard wait states: the asm must provide the 5 wait states
    between a VALU write of an SGPR (v_readfirstlane of the base and of the
    m0 value) and the VMEM instruction that reads it, and the 1 between an
    m0 write and the LDS DMA.  Without them a copy can read a stale base
    register and fetch from a wrong address.  A page's eight copies form one
    run: s_nop 4, then per copy an m0 write, s_nop 0 and the copy.  Launches
    with decode workers may also issue a tile's copies one at a time between
    the score MFMAs: runs of one, each with its own s_nop 4."""
    asm = _compile_to_asm(tmp_path)
    n, singles = 0, 0
    for name, body in _kernels(asm):
        fused = "ELb1ELb1E" in name  # <E, G, paged, decode workers>
        ins = [t for _, block in _blocks(body) for t in block]
        k = 0
        while k < len(ins):
            if not ins[k].startswith("s_nop 4"):
                k += 1
                continue
            run, j = 0, k + 1
            while j + 2 < len(ins) and re.match(r"s_(mov_b32|add_u32) m0,", ins[j]) \
                    and ins[j + 1].startswith("s_nop 0") and ins[j + 2].startswith("global_load_lds_dwordx4"):
                run += 1
                j += 3
            if run:
                assert run == 8 or (run == 1 and fused), (name, ins[k:j + 1])
                n += run
                singles += run == 1
            k = max(j, k + 1)
    total = sum(t.startswith("global_load_lds_dwordx4") for _, body in _kernels(asm)
                for _, block in _blocks(body) for t in block)
    # every copy sits in such a run; the six fused instantiations have single copies
    assert n == total and n >= 18 * 8, (n, total)
    assert singles >= 6 * 8, singles
