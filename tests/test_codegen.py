"""Code-generation guard for the streaming kernels (CPU only: hipcc cross-compiles).

The decode kernels run at the 256-register limit.  A register the compiler
spills and reloads inside a K/V streaming loop costs far more than the reload:
the scratch load is counted by vmcnt, which drains in issue order, so waiting
for it waits for every K/V block in flight (measured: config 2 B=1 loop end
21.7 -> 25.9 us).  Small source changes anywhere in the kernel can move a
spill into a loop, so this test compiles the device code to assembly and
checks that no scratch access sits in a basic block of a loop that also holds
MFMA instructions, for every decode-split and decode-layer kernel.
"""
import os
import re
import subprocess

import pytest

from supersonic_amd import build as B

KERNELS = re.compile(r"^(_ZN3ssa19decode_(?:split|layer)_kernel[^:\s]*):")
LOOP = re.compile(r"in Loop: Header=(BB\d+_\d+)")


def _asm(src, out_dir):
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [B.hipcc()] + B.HIP_FLAGS + ["-I", os.path.join(os.path.dirname(B.HERE), "include"),
                                       "--cuda-device-only", "-S", src, "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"asm failed: {' '.join(cmd)}\n{r.stderr[-4000:]}")
    return open(out).read().split("\n")


def loop_scratch(lines):
    """{kernel: [scratch instructions inside a loop that contains MFMAs]}"""
    found, name, blocks = {}, None, []
    for ln in lines + [".Lfunc_end_sentinel:"]:
        m = KERNELS.match(ln)
        if m or ln.startswith(".Lfunc_end"):
            if name is not None:
                mfma_loops = {h for h, ins in blocks if h and any("v_mfma" in i for i in ins)}
                bad = [i.strip() for h, ins in blocks if h in mfma_loops for i in ins if "scratch_" in i]
                found[name] = bad
            name, blocks = (m.group(1), [(None, [])]) if m else (None, [])
            continue
        if name is None:
            continue
        is_label = (ln.startswith(".LBB") and ln.split(";")[0].strip().endswith(":")) or ln.startswith("; %bb.")
        if is_label:
            lm = LOOP.search(ln)
            blocks.append((lm.group(1) if lm else None, []))
        elif ln.startswith("\t") and not ln.strip().startswith(";"):
            blocks[-1][1].append(ln.split(";")[0])
    return found


@pytest.mark.slow
@pytest.mark.parametrize("src", ["decode.hip", "layer.hip"])
def test_no_scratch_in_streaming_loops(tmp_path, src):
    found = loop_scratch(_asm(os.path.join(B.CSRC, src), str(tmp_path)))
    assert found, "no decode kernels found in the assembly"
    bad = {k: v for k, v in found.items() if v}
    assert not bad, f"scratch accesses inside MFMA loops: {bad}"


def test_loop_scratch_parser():
    """The parser on a hand-written listing: a spill reloaded inside an MFMA
    loop is found, one after the loop is not."""
    asm = """_ZN3ssa19decode_split_kernelIXEEvv:
\tv_mov_b32 v1, 0
\tscratch_store_dword off, v1, off
.LBB0_2:                                ;   in Loop: Header=BB0_2 Depth=1
\tv_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]
\tscratch_load_dword v2, off, off
\ts_cbranch_scc1 .LBB0_2
.LBB0_3:
\tscratch_load_dword v3, off, off
.Lfunc_end0:""".split("\n")
    found = loop_scratch(asm)
    assert list(found) == ["_ZN3ssa19decode_split_kernelIXEEvv"]
    assert found["_ZN3ssa19decode_split_kernelIXEEvv"] == ["scratch_load_dword v2, off, off"]


PREFILL = re.compile(r"^(_ZN3ssa14prefill_kernel[^:\s]*Li256[^:\s]*):")


def key_loop_read_ahead(lines):
    """{prefill kernel: K operand reads issued back to back ahead of the QK^T
    MFMAs}.  The source asks for kKLA (8) of them with a scheduling group whose
    marker the assembly listing keeps ("sched_group_barrier mask(0x00000100)
    size(8) SyncID(0)"); this counts the ds_read_b128 run that ends at the
    marker.  The compiler keeps the run only while it has the registers."""
    found, name, run = {}, None, 0
    for ln in lines:
        m = PREFILL.match(ln)
        if m:
            name, run = m.group(1), 0
            continue
        if name is None or name in found:
            continue
        ins = ln.strip()
        if "sched_group_barrier mask(0x00000100) size(8) SyncID(0)" in ins:
            found[name] = run
        elif ins.startswith("ds_read_b128"):
            run += 1
        elif ins and not ins.startswith(";"):
            run = 0
    return found


def test_key_loop_read_ahead_parser():
    """The parser on hand-written listings: eight reads ahead pass, a read
    interleaved with its MFMA is found."""
    head = "_ZN3ssa14prefill_kernelIXLi256EEvv:\n"
    marker = "\t; sched_group_barrier mask(0x00000100) size(8) SyncID(0)\n"
    good = head + "\ts_mul_i32 s1, s1, 0x10400\n" + "\tds_read_b128 v[0:3], v9\n" * 8 + marker
    bad = head + "\tds_read_b128 v[0:3], v9\n\ts_waitcnt lgkmcnt(0)\n\tv_mfma_f32_16x16x32_bf16 v[4:7], v[0:3], v[8:11], 0\n" \
        "\tds_read_b128 v[0:3], v9\n" + marker
    assert key_loop_read_ahead(good.split("\n")) == {"_ZN3ssa14prefill_kernelIXLi256EEvv": 8}
    assert key_loop_read_ahead(bad.split("\n")) == {"_ZN3ssa14prefill_kernelIXLi256EEvv": 1}


@pytest.mark.slow
def test_prefill_key_loop_reads_ahead(tmp_path):
    """The D=256 prefill kernels run at the register limit of three waves a
    SIMD; a few more values live across the key loop made the compiler issue
    one K read per MFMA instead of eight ahead (measured: 3060 -> 5350 cycles
    a key tile).  This checks the look-ahead in the assembly."""
    found = key_loop_read_ahead(_asm(os.path.join(B.CSRC, "prefill.hip"), str(tmp_path)))
    assert found, "no D=256 prefill kernels found in the assembly"
    bad = {k: v for k, v in found.items() if v < 8}
    assert not bad, f"K reads ahead of the first QK MFMA: {bad}"
