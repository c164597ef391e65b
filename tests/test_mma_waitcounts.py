"""Static check of the hand-counted vmcnt waits in mma.hip, on the AMD assembly of this build.

The M <= 64 kernel stages activation chunks and sidecars with direct-to-LDS buffer loads, which
the compiler does not track: the only thing that makes a stage's data visible in LDS before the
barrier that hands it to the other waves is an `s_waitcnt vmcnt(N)` whose N the source computes
by hand (kMidWait = 2 kWLoads + kStageLoads in the main loop; 2 kWLoads + 2 kStageLoads in the
prologue). N is only right if the compiler keeps the loads in the issue order the source assumes.
vmcnt counts down in issue order, and loads into LDS are never reordered among themselves (they
all may write LDS), so the condition is: at every barrier, the loads that may still be
outstanding (the N youngest before the last vmcnt wait, plus any loads into LDS issued after it) include at most
N - 2 kWLoads loads into LDS -- the stages the design leaves in flight. A compiler change that
sinks a stage's load below the weight loads it is counted against fails this test.

The worst case over the control-flow paths into a barrier is found by a memoised walk back over
the basic blocks, so branchy code costs no more than straight code. CPU only: hipcc cross-compiles
gfx950 to assembly here (about 10 s)."""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"

VMEM = re.compile(r"^\s*(buffer_load|global_load|buffer_store|global_store|buffer_atomic|global_atomic)")


def _kernels(asm, symbol=r"_ZN6splosh10mma_kernel\S*"):
    lines = asm.split("\n")
    starts = [i for i, l in enumerate(lines) if re.match(rf"^{symbol}:", l)]
    for j, i in enumerate(starts):
        # The function runs to its end label (it may have more than one s_endpgm).
        end = next((k for k in range(i, len(lines)) if lines[k].startswith(".Lfunc_end")), len(lines))
        code = []
        for l in lines[i + 1:end + 1]:
            m = re.search(r"; splosh-lds-outstanding (\d+)", l)
            code.append(f"#MARK {m.group(1)}" if m else l.split(";")[0].strip())
        yield lines[i].split(":")[0], code


def _weight_loads(name):
    """kWLoads of the instantiation, from its mangled template arguments."""
    m = re.search(r"Q4FormatILi(\d)ELb(\d)", name)
    if m:
        nw, tiled = int(m.group(1)), m.group(2) == "1"
        return nw if tiled else 3 * nw
    m = re.search(r"GgufFormatILi(\d+)E", name)
    if m:
        # gguf_fetch's buffer loads per format: fp16 fields and the dword windows of its spans.
        return {8: 4, 20: 3, 14: 8, 11: 9, 21: 7, 23: 4}[int(m.group(1))]
    m = re.search(r"Q5FormatILi\d+ELi\d+ELi\d+ELb(\d)", name)
    assert m, name
    return 2 if m.group(1) == "1" else 1


def _stage_loads(name):
    """Loads into LDS of one stage: the activation chunk (FM x 32 rows x KW x 8 pieces over CW x
    KW waves) plus one sidecar/meta load when those are staged (tiled q4, Q4_K/Q5_K)."""
    m = re.search(r"EELi(\d)ELi(\d)ELi(\d)ELi(\d)EEEvNS_7MmaArgsE", name)
    assert m, name
    fm, cw, kw = int(m.group(1)), int(m.group(2)), int(m.group(3))
    a_per = fm * 32 * kw * 8 // (cw * kw * 64)
    staged = bool(re.search(r"Q4FormatILi\dELb1", name)) or "Q5Format" in name
    return a_per + (1 if staged else 0)


def _cfg(code):
    """Basic blocks of a function: instruction lists and predecessor lists."""
    blocks, labels, cur = [], {}, []
    for ins in code:
        if not ins:
            continue
        if re.match(r"^\.LBB\d+_\d+:", ins):
            if cur:
                blocks.append(cur)
            cur = []
            labels[ins[:-1]] = len(blocks)
            continue
        cur.append(ins)
        if ins.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
            blocks.append(cur)
            cur = []
    if cur:
        blocks.append(cur)
    # Labels point at the block that starts after them.
    preds = [[] for _ in blocks]
    for b, ins_list in enumerate(blocks):
        last = ins_list[-1] if ins_list else ""
        tgt = re.match(r"^s_c?branch\S*\s+(\.LBB\d+_\d+)", last)
        if tgt and tgt.group(1) in labels:
            preds[labels[tgt.group(1)]].append(b)
        if not last.startswith(("s_branch", "s_endpgm", "s_setpc")) and b + 1 < len(blocks):
            preds[b + 1].append(b)
    return blocks, preds


def _is_lds(ins):
    return ins.startswith("buffer_load") and ins.endswith(" lds")


def _max_lds(blocks, preds, b, idx, want, memo, stack):
    """The most loads into LDS among the `want` youngest VMEM instructions issued before
    instruction idx of block b, over every path of predecessors (a path that reaches the function
    entry, or closes a cycle without enough loads, ends there). Memoised per (block, count), so
    branchy code does not multiply the paths."""
    got = lds = 0
    for ins in reversed(blocks[b][:idx]):
        if got == want:
            return lds
        if VMEM.match(ins):
            got += 1
            lds += _is_lds(ins)
    if got == want or not preds[b]:
        return lds
    best = 0
    for p in preds[b]:
        key = (p, want - got)
        if key in stack:
            continue
        if key not in memo:
            stack.add(key)
            memo[key] = _max_lds(blocks, preds, p, len(blocks[p]), want - got, memo, stack)
            stack.discard(key)
        best = max(best, memo[key])
    return lds + best


def _check_function(name, code, stage=None):
    """Checks every barrier after a vmcnt wait; returns (barriers with loads into LDS allowed to
    stay in flight, barriers checked)."""
    stage = _stage_loads(name) if stage is None else stage
    blocks, preds = _cfg(code)
    checked = waited = 0
    memo = {}
    for b, ins_list in enumerate(blocks):
        for i, ins in enumerate(ins_list):
            if not ins.startswith("s_barrier"):
                continue
            # The design's statement, if any: "; splosh-lds-outstanding K" (comments are stripped
            # from `code`, so look in the raw marker list kept beside it).
            allowed = 0
            for k in range(i - 1, max(i - 4, -1), -1):
                m = re.match(r"^#MARK (\d+)$", ins_list[k])
                if m:
                    allowed = int(m.group(1))
                    break
            # The last vmcnt wait before this barrier in the block, and VMEM issued since.
            after, n, wait_at = 0, None, None
            for k in range(i - 1, -1, -1):
                m = re.search(r"vmcnt\((\d+)\)", ins_list[k]) if ins_list[k].startswith("s_waitcnt") else None
                if m:
                    n, wait_at = int(m.group(1)), k
                    break
                if VMEM.match(ins_list[k]) and _is_lds(ins_list[k]):
                    after += 1
            if n is None:
                continue
            waited += 1
            lds = _max_lds(blocks, preds, b, wait_at, n, memo, set()) + after
            assert lds <= allowed, (
                f"{name}: a barrier's vmcnt({n}) leaves {lds} loads into LDS outstanding, the "
                f"design allows {allowed}")
            if allowed:
                assert allowed % stage == 0, (name, allowed, stage)
                checked += 1
    return checked, waited


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="needs hipcc")
def test_mma_stage_waits_cover_their_loads(tmp_path):
    out = tmp_path / "mma.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", "--cuda-device-only", "-S",
           str(ROOT / "splosh_amd" / "csrc" / "mma.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    kernels = list(_kernels(out.read_text()))
    assert len(kernels) >= 8
    for name, code in kernels:
        # Every instantiation has the prologue barrier and at least three mid-step barriers whose
        # waits keep loads in flight.
        assert _check_function(name, code)[0] >= 4, name


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="needs hipcc")
def test_prefill_stage_waits_cover_their_loads(tmp_path):
    """The prefill kernel's activations arrive through loads into LDS, four a wave and group; the
    wait before each step's barrier must leave none of them in flight (only the weight loads issued
    after them), for every weight format it stages."""
    out = tmp_path / "prefill.s"
    cmd = [HIPCC, "-O3", "-std=c++17", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", f"-I{ROOT / 'include'}", "--cuda-device-only", "-S",
           str(ROOT / "splosh_amd" / "csrc" / "prefill.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    kernels = list(_kernels(out.read_text(), r"_ZN6splosh14prefill_kernel\S*"))
    assert len(kernels) == 10  # q4, fused q4 gate+up, Q5_K, Q4_K and the six native GGUF formats
    for name, code in kernels:
        assert any(_is_lds(ins) for ins in code), name
        # The prologue's barrier and the two unrolled steps'.
        assert _check_function(name, code, stage=4)[1] >= 3, name
