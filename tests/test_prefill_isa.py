"""The prefill GEMM's weight loads are inline asm whose results the compiler believes ready at once; the kernel
waits for them itself, by count, at the top of the stage that reads them (three stages later). That is sound only
if the compiled code touches none of those registers in between: no copy, no spill, no reuse. This test compiles
kernels_prefill.hip for gfx950 to assembly and checks exactly that, for every loop of both GEMM kernels, and
that the loads issued before a loop are not touched before that loop's first wait. Needs hipcc (no GPU)."""
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "vitna-anchor_amd", "csrc", "kernels_prefill.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# the stage-top waits (2 NA + 2 NB loads may run, NA = 8, 4, 2 for 256-, 128- and 64-row tiles) and the stages a
# weight load stays in flight
WAITS = {36, 28, 24}
LEAD = 3


def regs(op):
    m = re.match(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", op)
    return {int(m.group(1))} if m else set()


def used(ins):
    if " " not in ins:
        return set()
    out = set()
    for o in ins.split(None, 1)[1].split(","):
        out |= regs(o.strip())
    return out


def is_top(ins):
    m = re.match(r"s_waitcnt vmcnt\((\d+)\)$", ins)
    return bool(m) and int(m.group(1)) in WAITS


def check_kernel(lines):
    problems = []
    heads = [i for i, l in enumerate(lines) if l.startswith(".LBB") and "Loop Header" in l]
    code = [l.strip() for l in lines]
    loops = 0
    for h in heads:
        lab = lines[h].split(":")[0]
        end = next(i for i in range(h + 1, len(lines)) if re.search(r"s_cbranch\w*\s+" + re.escape(lab) + r"\b", lines[i]))
        body = [c for c in code[h + 1:end + 1] if c and not c.startswith(";") and not c.startswith(".")]
        tops = [i for i, c in enumerate(body) if is_top(c)]
        if not tops:
            continue
        loops += 1
        n = len(body)
        for i, c in enumerate(body):
            if not re.match(r"global_load_dword(x2)?\s", c):
                continue
            dst = regs(c.split()[1].rstrip(","))
            seen = 0
            for step in range(1, 4 * n):
                ins = body[(i + step) % n]
                if is_top(ins):
                    seen += 1
                    if seen == LEAD:
                        break
                elif used(ins) & dst:
                    problems.append("%s: %s touched by %s after %d waits" % (lab, c, ins, seen))
                    break
        # loads before the loop: untouched until the loop's first stage-top wait
        p0 = max(i for i in range(h) if code[i].startswith("s_waitcnt vmcnt(0)"))
        for i in range(p0, h):
            if not re.match(r"global_load_dword(x2)?\s", code[i]):
                continue
            dst = regs(code[i].split()[1].rstrip(","))
            for k in range(i + 1, len(code)):
                ins = code[k]
                if is_top(ins):
                    break
                if ins and not ins.startswith((";", ".")) and used(ins) & dst:
                    problems.append("before %s: %s touched by %s" % (lab, code[i], ins))
                    break
    return loops, problems


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_weight_registers_untouched_until_waited():
    tmp = tempfile.mkdtemp()
    try:
        out = os.path.join(tmp, "k.s")
        subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
                        "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang",
                        "-packed-fp32-ops", "--cuda-device-only", "-S", SRC, "-o", out], check=True, capture_output=True)
        text = open(out).read().splitlines()
        for gu in ("1", "0"):
            name = "_Z20prefill_wgemm_kernelILb%sEEv12prefill_args:" % gu
            start = next(i for i, l in enumerate(text) if l.startswith(name))
            stop = next(i for i in range(start, len(text)) if text[i].strip() == "s_endpgm")
            loops, problems = check_kernel(text[start:stop + 1])
            assert loops == 3, (gu, loops)  # the 256-, 128- and 64-row tiles
            assert not problems, problems[:5]
    finally:
        shutil.rmtree(tmp)


def test_checker_catches_an_early_touch():
    """The checker itself: a loop whose weight register is copied before its third stage-top wait is caught, the
    same loop without the copy passes."""
    good = [
        "s_waitcnt vmcnt(0)",
        ".LBB0_1:                                ; =>This Inner Loop Header: Depth=1",
        "s_waitcnt vmcnt(36)",
        "global_load_dwordx2 v[10:11], v[4:5], off",
        "s_waitcnt vmcnt(36)",
        "v_add_u32_e32 v1, v2, v3",
        "s_waitcnt vmcnt(36)",
        "s_waitcnt vmcnt(36)",
        "v_add_u32_e32 v1, v10, v3",
        "s_cbranch_scc0 .LBB0_1",
    ]
    assert check_kernel(good) == (1, [])
    bad = list(good)
    bad.insert(5, "v_mov_b32_e32 v20, v11")
    loops, problems = check_kernel(bad)
    assert loops == 1 and len(problems) == 1 and "v_mov_b32_e32 v20, v11" in problems[0]
