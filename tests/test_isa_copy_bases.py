"""CPU: the HBM -> LDS copies of the decode and prefill kernels read SGPR bases that no VALU
instruction wrote shortly before.

A `global_load_lds_*` whose SGPR base a `v_readfirstlane` had written 5 wait states earlier
copied from a wrong base now and then on gfx950: the q8_0 decode kernel returned whole KV heads
wrong or NaN at 16K keys. The kernels make each cache base uniform once (`sgpr_base`, padded with
18 wait states) and add block offsets with SALU instructions (`sgpr_offset`). This test compiles
decode.hip and prefill.hip to gfx950 assembly with the library's flags and checks every copy: the
last instruction before it (in program order, across labels) that writes one of its base SGPRs
is either not a VALU instruction, or is followed by at least 18 wait states before the copy.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "brasa_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
MIN_WAIT_STATES = 18
SCAN = 200  # instructions looked back per copy
# VALU instructions with an SGPR destination in their second operand (carry / condition out)
VOP3B = re.compile(r"v_(mad_u64_u32|mad_i64_i32|add_co_u32|sub_co_u32|subrev_co_u32|addc_co_u32|"
                   r"subb_co_u32|subbrev_co_u32|div_scale_f32|div_scale_f64)")

pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")


def _sgprs(op: str) -> set[int]:
    op = op.strip().split()[0] if op.strip() else ""
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m[1]), int(m[2]) + 1))
    m = re.fullmatch(r"s(\d+)", op)
    return {int(m[1])} if m else set()


def _written(mnemonic: str, ops: list[str]) -> set[int]:
    if not ops:
        return set()
    w = _sgprs(ops[0])
    if VOP3B.match(mnemonic) and len(ops) > 1:
        w |= _sgprs(ops[1])
    return w


def copy_base_hazards(asm: str) -> tuple[int, list[str]]:
    """(number of SGPR-based copies, descriptions of the ones whose base a VALU instruction
    wrote fewer than MIN_WAIT_STATES wait states before)."""
    lines = [l.split(";")[0].strip() for l in asm.splitlines()]
    n, bad, fn = 0, [], "?"
    for i, line in enumerate(lines):
        if line.endswith(":") and line.startswith("_Z"):
            fn = line[:-1]
        if not line.startswith("global_load_lds"):
            continue
        ops = line.split(None, 1)[1].split(",") if " " in line else []
        want = _sgprs(ops[1]) if len(ops) > 1 else set()
        if not want:
            continue
        n += 1
        ws = 0
        seen = 0
        for j in range(i - 1, -1, -1):
            t = lines[j]
            if not t or t.startswith(".") or t.endswith(":"):
                continue
            seen += 1
            if seen > SCAN:
                break
            parts = t.split(None, 1)
            mn = parts[0]
            if mn == "s_nop":
                ws += int(parts[1], 0) + 1
                continue
            ops_j = parts[1].split(",") if len(parts) > 1 else []
            hit = _written(mn, ops_j) & want
            if hit and not mn.startswith(("global_", "buffer_", "s_waitcnt")):
                if mn.startswith("v_") and ws < MIN_WAIT_STATES:
                    bad.append(f"{fn}: line {i + 1} `{line}` <- `{t}` after {ws} wait states")
                    break
                want = want - hit  # each register's last writer decides for it
                if not want:
                    break
            ws += 1
    return n, bad


def _compile(src: str, out: str) -> None:
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only",
           "-S", "-I", os.path.join(ROOT, "include"), os.path.join(CSRC, src), "-o", out]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)


@pytest.fixture(scope="module")
def kernels_asm(tmp_path_factory):
    d = tmp_path_factory.mktemp("isa")
    srcs = ["decode.hip", "prefill.hip"]
    outs = [str(d / (s + ".s")) for s in srcs]
    with ThreadPoolExecutor(2) as ex:
        list(ex.map(_compile, srcs, outs))
    yield {s: open(o).read() for s, o in zip(srcs, outs)}
    shutil.rmtree(d, ignore_errors=True)


@pytest.mark.parametrize("src", ["decode.hip", "prefill.hip"])
def test_copy_bases_not_fresh_valu_writes(kernels_asm, src):
    n, bad = copy_base_hazards(kernels_asm[src])
    assert n > 0, f"{src}: no SGPR-based LDS copies found (the scan no longer matches the ISA)"
    assert not bad, f"{src}: {len(bad)} of {n} copies:\n" + "\n".join(bad[:10])


def test_scan_flags_a_fresh_readfirstlane():
    """The scan itself: a base written by v_readfirstlane 5 wait states before the copy is
    flagged, the same base with 18 is not, an SALU-written base is not, and a pair with one
    half written by each is."""
    fresh = """_Zk:
    v_readfirstlane_b32 s3, v37
    v_readfirstlane_b32 s2, v36
    s_mov_b32 s7, m0
    s_mov_b32 m0, s20
    s_nop 2
    global_load_lds_dwordx4 v75, s[2:3] nt
"""
    padded = fresh.replace("s_nop 2", "s_nop 7\n s_nop 7\n s_nop 0")
    salu = """_Zk:
    v_readfirstlane_b32 s3, v37
    s_add_u32 s2, s4, s6
    s_addc_u32 s3, s5, s7
    global_load_lds_dwordx4 v75, s[2:3] nt
"""
    split = """_Zk:
    v_readfirstlane_b32 s2, v36
    s_mov_b32 s3, s9
    global_load_lds_dwordx4 v75, s[2:3] nt
"""
    carry = """_Zk:
    v_mad_u64_u32 v[34:35], s[2:3], s10, v34, v[122:123]
    global_load_lds_dword v75, s[2:3]
"""
    n, bad = copy_base_hazards(fresh)
    assert n == 1 and len(bad) == 1
    assert copy_base_hazards(padded) == (1, [])
    assert copy_base_hazards(salu) == (1, [])
    assert len(copy_base_hazards(split)[1]) == 1
    assert len(copy_base_hazards(carry)[1]) == 1
