"""ISA checks of the gfx950 kernels (CPU: hipcc cross-compiles, nothing runs).

The MFMA paths read LDS with inline asm (the compiler would otherwise wait for
every direct global->LDS load before each LDS read) and wait with explicit
s_waitcnt.  The compiler does not know those reads are asynchronous, so it may
schedule a copy of a destination register before the wait -- a wrong-result bug
the decode kernel once had.  These tests compile every kernel source to
assembly and check, on the code actually generated:

  * no instruction touches a register of an LDS read before an s_waitcnt
    lgkmcnt(N) has retired that read (LDS operations complete in order);
  * no instruction other than an MFMA accumulating into the same registers
    reads or writes an MFMA's destination sooner than the wait states the
    compiler itself keeps after its MFMAs (8 after a 16x16, 12 after a 32x32),
    along every control-flow path (loop exits included).
"""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "unillm_amd", "csrc")
SOURCES = ["decode.hip", "prefill.hip", "gemv.hip", "weights.hip", "attention.hip"]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature",
         "-Xclang", "-packed-fp32-ops", "-S", "--cuda-device-only"]


def _hipcc():
    for c in ("/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    hipcc = _hipcc()
    if not hipcc:
        pytest.skip("hipcc not available")
    out = {}
    d = tmp_path_factory.mktemp("isa")
    for src in SOURCES:
        path = str(d / (src + ".s"))
        subprocess.run([hipcc, *FLAGS, os.path.join(CSRC, src), "-o", path], check=True,
                       capture_output=True)
        out[src] = open(path).read()
    return out


def _regs(tok):
    m = re.match(r"([vas])\[(\d+):(\d+)\]", tok)
    if m:
        return {f"{m.group(1)}{i}" for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    return {tok} if re.match(r"[vas]\d+$", tok) else set()


def _ops(line):
    return [o for o in re.split(r"[ ,]+", line) if o]


def _functions(text):
    """(name, [instructions], {label: index}) per kernel, comments stripped."""
    funcs, cur = [], None
    for raw in text.split("\n"):
        line = raw.split(";")[0].strip()
        if not line:
            continue
        m = re.match(r"^(_Z\S+|[A-Za-z_]\w*):$", line)
        if m and not line.startswith("."):
            cur = (m.group(1), [], {})
            funcs.append(cur)
            continue
        if cur is None:
            continue
        if re.match(r"^\.LBB\S+:$", line):
            cur[2][line[:-1]] = len(cur[1])
            continue
        if line.startswith("."):
            continue
        cur[1].append(line)
    return [f for f in funcs if f[1]]


def lds_read_hazards(text):
    """Registers of an LDS read touched before an lgkmcnt wait retires the read
    (straight-line code between labels; LDS ops complete in order)."""
    bad = []
    for name, ins, labels in _functions(text):
        label_at = set(labels.values())
        queue = []  # destination registers of outstanding LDS / scalar-memory ops, oldest first
        for k, line in enumerate(ins):
            if k in label_at:
                queue = []
            m = re.match(r"s_waitcnt.*lgkmcnt\((\d+)\)", line)
            if m:
                n = int(m.group(1))
                queue = queue[len(queue) - n:] if 0 < n < len(queue) else ([] if n == 0 else queue)
                continue
            if line.startswith("s_waitcnt"):
                continue
            o = _ops(line)
            pending = set().union(*queue) if queue else set()
            if o[0].startswith(("ds_read", "s_load", "s_buffer_load")):
                srcs = set().union(*[_regs(x) for x in o[2:]]) if len(o) > 2 else set()
                if srcs & pending:
                    bad.append(f"{name}: {line}")
                queue.append(_regs(o[1]) if o[0].startswith("ds_read") else set())
                continue
            if o[0].startswith("ds_"):
                queue.append(set())
            touched = set().union(*[_regs(x) for x in o[1:]]) if len(o) > 1 else set()
            if touched & pending:
                bad.append(f"{name}: {line}")
    return bad


def mfma_result_hazards(text):
    """Readers or writers of an MFMA destination within the wait states the
    compiler keeps after its own MFMAs, along all control-flow paths."""
    bad = []
    for name, ins, labels in _functions(text):
        for k, line in enumerate(ins):
            if not line.startswith("v_mfma"):
                continue
            o = _ops(line)
            dst = _regs(o[1])
            need = 12 if "32x32" in o[0] else 8
            stack, seen = [(k + 1, need)], set()
            while stack:
                p, w = stack.pop()
                while 0 <= p < len(ins) and w > 0 and (p, w) not in seen:
                    seen.add((p, w))
                    t = ins[p]
                    to = _ops(t)
                    if t.startswith("v_mfma"):
                        if set().union(*[_regs(x) for x in to[2:4]]) & dst:
                            bad.append(f"{name}: {line} -> {t}")
                        if _regs(to[1]) == dst:
                            break  # accumulating into the same registers: the hardware chains it
                    elif (set().union(*[_regs(x) for x in to[1:]]) if len(to) > 1 else set()) & dst:
                        bad.append(f"{name}: {line} -> {t}")
                        break
                    m = re.match(r"s_nop (\d+)", t)
                    w -= int(m.group(1)) + 1 if m else 1
                    if t.startswith("s_endpgm"):
                        break
                    m = re.match(r"s_(branch|cbranch_\w+)\s+(\S+)", t)
                    if m:
                        if m.group(2) in labels:
                            stack.append((labels[m.group(2)], w))
                        if m.group(1) == "branch":
                            break
                    p += 1
    return bad


@pytest.mark.parametrize("src", SOURCES)
def test_lds_reads_waited_before_use(asm, src):
    assert lds_read_hazards(asm[src]) == []


@pytest.mark.parametrize("src", SOURCES)
def test_mfma_results_not_read_early(asm, src):
    assert mfma_result_hazards(asm[src]) == []


def test_checkers_catch_planted_hazards():
    # the checkers themselves: a copy of an LDS result before its wait, and an
    # accumulator read right after the MFMA that writes it
    lds = "k:\n ds_read_b128 v[4:7], v1\n v_mov_b32 v8, v5\n s_waitcnt lgkmcnt(0)\n s_endpgm\n"
    assert len(lds_read_hazards(lds)) == 1
    ok = "k:\n ds_read_b128 v[4:7], v1\n s_waitcnt lgkmcnt(0)\n v_mov_b32 v8, v5\n s_endpgm\n"
    assert lds_read_hazards(ok) == []
    mf = ("k:\n v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]\n s_branch .LBB0_1\n"
          ".LBB0_1:\n v_accvgpr_read_b32 v9, a1\n s_endpgm\n")
    assert len(mfma_result_hazards(mf)) == 1
    mf_ok = mf.replace(" s_branch .LBB0_1\n", " s_nop 7\n s_branch .LBB0_1\n")
    assert mfma_result_hazards(mf_ok) == []
