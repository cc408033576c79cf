"""CPU: two properties of the generated gfx950 code of the decode and prefill kernels that the
compiler does not check for inline asm.

1. The HBM -> LDS copies read SGPR bases that no VALU instruction wrote shortly before.
   A `global_load_lds_*` whose SGPR base a `v_readfirstlane` had written 5 wait states earlier
   copied from a wrong base now and then on gfx950: the q8_0 decode kernel returned whole KV
   heads wrong or NaN at 16K keys. The kernels make each cache base uniform once (`sgpr_base`,
   padded with 18 wait states) and add block offsets with SALU instructions (`sgpr_offset`).
   Checked for every copy: the last instruction before it (in program order, across labels)
   that writes one of its base SGPRs is either not a VALU instruction, or is followed by at
   least 18 wait states before the copy.
2. In each kernel's prologue, no instruction reads or overwrites a VGPR that an inline-asm load
   is still to write. Such a load writes its registers when the data returns; the compiler
   treats them as written at the asm, so only an `s_waitcnt vmcnt` (and an asm naming the
   registers after it) keeps it from copying or reusing them early. A wait chosen by a branch
   once let it copy the Q registers of the q8_0 decode kernel before the wait. Checked on every
   path of the control flow graph from the kernel's entry to that path's first vmcnt wait:
   every VGPR operand against the destinations of the inline-asm loads issued on the path.
   (Past that point the ring loops' waits depend on the block count through EXEC-masked
   branches, whose impossible paths a static scan cannot tell apart.)
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
MAX_STATES = 256  # distinct pending-load lists kept per basic block
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


def _vgprs(op: str) -> frozenset:
    op = op.strip().split()[0] if op.strip() else ""
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", op)
    if m:
        return frozenset(range(int(m[1]), int(m[2]) + 1))
    m = re.fullmatch(r"v(\d+)", op)
    return frozenset({int(m[1])}) if m else frozenset()


def _functions(asm: str) -> dict:
    """Kernel name -> [(line, instruction)], inline-asm instructions prefixed with '@'."""
    fns, cur, in_asm = {}, None, False
    for ln, raw in enumerate(asm.splitlines(), 1):
        if "ASMSTART" in raw:
            in_asm = True
            continue
        if "ASMEND" in raw:
            in_asm = False
            continue
        t = raw.split(";")[0].strip()
        if not t or (t.startswith(".") and not t.endswith(":")):
            continue
        if t.endswith(":") and t.startswith("_Z"):
            cur = t[:-1]
            fns[cur] = []
            continue
        if cur is None:
            continue
        if t.startswith(".Lfunc_end"):
            cur = None
            continue
        fns[cur].append((ln, "@" + t if in_asm and not t.endswith(":") else t))
    return fns


def _inflight_uses(lines: list, maxdepth: int = 64) -> dict:
    # basic blocks: a label starts one, a branch ends one
    blocks, cur = [], ("", [])
    for ln, t in lines:
        if t.endswith(":"):
            blocks.append(cur)
            cur = (t[:-1], [])
            continue
        cur[1].append((ln, t))
        if t.lstrip("@").startswith(("s_branch", "s_cbranch")):
            blocks.append(cur)
            cur = (f"<after {ln}>", [])
    blocks.append(cur)
    index = {b[0]: i for i, b in enumerate(blocks)}
    succ = []
    for i, (_, ins) in enumerate(blocks):
        s, fall = [], True
        for _, t in ins:
            w = t.lstrip("@").split()
            if w[0] == "s_branch":
                s.append(index.get(w[1]))
                fall = False
            elif w[0] == "s_cbranch_execz":
                # taken only when no lane would run the skipped code: for the uniform conditions
                # of these kernels the code is then a no-op, so only the fall-through is followed
                # (the pending loads can only be overcounted)
                pass
            elif w[0].startswith("s_cbranch"):
                s.append(index.get(w[1]))
            elif w[0] == "s_endpgm":
                fall = False
        if fall and i + 1 < len(blocks):
            s.append(i + 1)
        succ.append([x for x in s if x is not None])

    # Each block keeps the set of distinct pending lists that reach it (the paths are tracked
    # separately, so two branches that skip each other's loads do not blur the counts); past
    # MAX_STATES lists, they are merged from the newest end (an over-approximation).
    def merge_all(states):
        n = max(len(x) for x in states)
        pads = [(frozenset(),) * (n - len(x)) + x for x in states]
        return tuple(frozenset().union(*col) for col in zip(*pads))[-maxdepth:]

    state = [frozenset() for _ in blocks]
    state[0] = frozenset({()})
    work, hits = [0], {}
    while work:
        i = work.pop()
        outs = set()
        for start_st in state[i]:
            st = list(start_st)
            stopped = False
            for ln, t in blocks[i][1]:
                asm = t.startswith("@")
                t = t.lstrip("@")
                parts = t.split(None, 1)
                mn = parts[0]
                ops = parts[1].split(",") if len(parts) > 1 else []
                if mn == "s_waitcnt":
                    m = re.search(r"vmcnt\((\d+)\)", t)
                    if m:
                        stopped = True  # the prologue ends at a path's first vmcnt wait
                        break
                    continue
                is_load = (bool(re.match(r"(global|buffer|flat|scratch)_load_", mn))
                           and "_lds_" not in mn)
                is_vmem = bool(re.match(r"(global|buffer|flat|scratch)_(load|store|atomic)", mn))
                writes_first = (mn.startswith("v_") or is_load or mn.startswith(("ds_read", "ds_load"))
                                ) and not mn.startswith(("global_store", "buffer_store"))
                regs = set()
                dst = frozenset()
                for k, o in enumerate(ops):
                    r = _vgprs(o)
                    if k == 0 and writes_first:
                        dst |= r
                    regs |= r
                for reg, origin in (frozenset().union(*st) if st else frozenset()):
                    if reg in regs:
                        hits.setdefault(ln, (t, origin))
                if is_vmem:
                    st.append(frozenset((r, ln) for r in dst) if is_load and asm else frozenset())
                st = st[-maxdepth:]
            if not stopped:
                outs.add(tuple(st))
        for j in succ[i]:
            new = state[j] | outs
            if len(new) > MAX_STATES:
                new = frozenset({merge_all(list(new))})
            if new != state[j]:
                state[j] = new
                work.append(j)
    return hits


def inflight_register_uses(asm: str) -> list:
    """Descriptions of instructions that touch a VGPR a pending inline-asm load will write,
    from each kernel's entry to each path's first vmcnt wait."""
    bad = []
    for fn, lines in _functions(asm).items():
        for ln, (t, origin) in sorted(_inflight_uses(lines).items()):
            bad.append(f"{fn}: line {ln} `{t}` touches a register of the asm load at line {origin}")
    return bad


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


@pytest.mark.parametrize("src", ["decode.hip", "prefill.hip"])
def test_no_register_of_an_inflight_asm_load_touched_in_prologue(kernels_asm, src):
    bad = inflight_register_uses(kernels_asm[src])
    assert not bad, f"{src}: {len(bad)} instructions:\n" + "\n".join(bad[:10])


def test_inflight_scan_on_small_cases():
    """A copy of an asm-loaded register before the first wait is flagged, one after it is not,
    the compiler's own loads are not checked, and a branch around the wait is followed."""
    head = "_Zk:\n    ;;#ASMSTART\n    global_load_dwordx4 v[2:5], v[0:1], off\n    ;;#ASMEND\n"
    early = head + "    v_mov_b32_e32 v9, v3\n    s_waitcnt vmcnt(0)\n    s_endpgm\n"
    late = head + "    s_waitcnt vmcnt(0)\n    v_mov_b32_e32 v9, v3\n    s_endpgm\n"
    overwrite = head + "    v_mov_b32_e32 v4, 0\n    s_waitcnt vmcnt(0)\n    s_endpgm\n"
    compiler = ("_Zk:\n    global_load_dwordx4 v[2:5], v[0:1], off\n    v_mov_b32_e32 v9, v3\n"
                "    s_endpgm\n")
    branch = (head + "    s_cbranch_scc1 .LBB0_2\n    s_waitcnt vmcnt(0)\n.LBB0_2:\n"
              "    v_mov_b32_e32 v9, v3\n    s_endpgm\n")
    assert len(inflight_register_uses(early)) == 1
    assert inflight_register_uses(late) == []
    assert len(inflight_register_uses(overwrite)) == 1
    assert inflight_register_uses(compiler) == []
    assert len(inflight_register_uses(branch)) == 1


PROBE = r'''
#include <hip/hip_runtime.h>
typedef __attribute__((address_space(3))) void lds_t;
__global__ void probe(const float* const* __restrict__ pp, float* out) {
  __shared__ float sm[1024];
  const float* p = pp[threadIdx.x & 1];  // a pointer held in VGPRs
  const unsigned long long v = (unsigned long long)p;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
  const float* base = (const float*)(((unsigned long long)hi << 32) | lo);
  __builtin_amdgcn_global_load_lds((const void*)(base + threadIdx.x), (lds_t*)sm, 4, 0, 0);
  __syncthreads();
  out[threadIdx.x] = sm[threadIdx.x ^ 1];
}
'''


def test_compiler_pads_the_documented_hazard(tmp_path):
    """The published gfx9 hazard for a VALU write of an SGPR read by a vector memory instruction
    is 5 wait states; the gfx950 compiler's own hazard recognizer pads exactly that (s_nop 4)
    between v_readfirstlane and a compiler-generated global_load_lds with that SGPR base. The
    inline-asm copies of the kernels failed with 5 and are held to MIN_WAIT_STATES (18), an
    empirical margin above the documented requirement, not a documented figure."""
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    out = tmp_path / "probe.s"
    _compile(str(src), str(out))
    asm = out.read_text()
    body = asm[asm.index("probe"):]
    lines = [l.split(";")[0].strip() for l in body.splitlines()]
    i = max(k for k, l in enumerate(lines) if l.startswith("v_readfirstlane_b32"))
    j = next(k for k in range(i, len(lines)) if lines[k].startswith("global_load_lds"))
    states = 0
    for l in lines[i + 1:j]:
        m = re.match(r"s_nop\s+(\d+)", l)
        states += int(m[1]) + 1 if m else (1 if l and not l.endswith(":") else 0)
    assert states == 5, (states, lines[i:j + 1])
    assert MIN_WAIT_STATES > states
