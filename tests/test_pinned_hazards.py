"""The 4-wave GEMM issues its MFMAs as inline asm with the accumulator
tied in AGPRs, and the skinny GEMM with the accumulator tied in VGPRs;
the compiler's hazard tracking does not see into either.  This compiles
the kernels to gfx950 assembly (no GPU needed) and checks, for every such
kernel, what that tracking would otherwise guarantee:
  - no VALU instruction writes an MFMA source register within the
    2 wait states before the MFMA reads it;
  - the main loop moves no accumulator (no copy between MFMAs);
  - every MFMA result is followed by at least 19 wait states (s_nop) before
    anything outside the MFMAs touches an accumulator, and the zeroing of
    the accumulators precedes the first MFMA by at least 2."""
import pathlib
import re
import shutil
import subprocess

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
PKG = REPO / "vpipe-sensenova-u1.5_amd"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _regs(spec):
    m = re.match(r"([va])\[(\d+):(\d+)\]", spec)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", spec)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _wait_states(line):
    return int(line.split()[1]) + 1 if line.startswith("s_nop") else 1


@pytest.fixture(scope="module")
def kernels():
    if not pathlib.Path(HIPCC).exists():
        pytest.skip("hipcc not available")
    out = subprocess.run(
        [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17",
         "-Wno-unused-command-line-argument",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         f"-I{REPO / 'include'}", f"-I{PKG / 'csrc'}", "--cuda-device-only", "-S",
         str(PKG / "csrc" / "u15h_kernels.hip"), "-o", "-"],
        capture_output=True, text=True, timeout=600, check=True).stdout
    found = {}
    name = None
    for raw in out.splitlines():
        if re.match(r"^_Z\S*(mot_gemm_kernel\S*Li2E|skinny_(?:reg|lds|dma)_kernel)\S*:", raw):
            name = raw.split(":")[0]
            found[name] = []
            continue
        if name is not None:
            if raw.strip().startswith(".amdhsa_kernel") or raw.startswith(".Lfunc_end"):
                name = None
                continue
            s = raw.strip()
            if s and not s.startswith(";") and not s.startswith(".") and not s.endswith(":"):
                found[name].append(s)
    assert found, "no pinned-MFMA kernels in the assembly"
    return found


def test_every_epilogue_has_a_pinned_kernel(kernels):
    # 4-wave GEMM: bf16, SwiGLU, int32 and dequant epilogues, 256 MFMAs
    # each; skinny GEMM: the five row-group builds (register kernel for 16
    # rows, LDS kernel for 32, 64, 96 and 128) for bf16 weights and 4- and
    # 8-bit packs, with the DMA kernel for 16 rows of bf16 weights and the
    # 32-column-wave builds for 96 and 128 rows of bf16 weights: 2 MFMAs
    # (k-steps) per 16 rows, 16 columns and unrolled K-block, 2 blocks
    # unrolled in the register and DMA kernels, D (the ring depth) in the
    # LDS kernels
    four = [n for n in kernels if "mot_gemm_kernel" in n]
    skinny = [n for n in kernels if "skinny_" in n]
    assert len(four) == 4 and len(skinny) == 18
    for n in four:
        assert sum(1 for s in kernels[n] if s.startswith("v_mfma")) == 256
    for n in skinny:
        m = re.search(r"skinny_(reg|lds|dma)_kernelILi(\d+)E(?:Li(\d+)ELi\d+E(?:Li(\d+)E)?)?", n)
        mt = int(m.group(2))
        depth = int(m.group(3)) if m.group(1) == "lds" else 2
        cw = int(m.group(4)) if m.group(4) else 1    # 16-column fragments per wave
        assert sum(1 for s in kernels[n] if s.startswith("v_mfma")) == 2 * mt * depth * cw


def _operands(s):
    return [o.strip() for o in s.split(None, 1)[1].split(",")] if " " in s else []


def _acc_regs(body):
    """Every register an MFMA of the body accumulates in."""
    regs = set()
    for s in body:
        if s.startswith("v_mfma"):
            regs |= _regs(_operands(s)[0])
    return regs


def _touches(s, regs):
    return any(_regs(o) & regs for o in _operands(s))


def _valu_hazards(body):
    """VALU writes of an MFMA source register within 2 wait states of it."""
    bad = []
    for i, s in enumerate(body):
        if not s.startswith("v_mfma"):
            continue
        srcs = set().union(*(_regs(o) for o in _operands(s)[1:]))
        ws, k = 0, i - 1
        while k >= 0 and ws < 2:
            p = body[k]
            op = p.split()[0]
            if op.startswith("v_") and not op.startswith("v_mfma"):
                if _regs(_operands(p)[0]) & srcs:
                    bad.append((p, ws, s))
            ws += _wait_states(p)
            k -= 1
    return bad


def _unsettled_acc_read(body):
    """The first access of an accumulator register after the last MFMA
    with fewer than 19 wait states between them, or None."""
    acc = _acc_regs(body)
    last = max(i for i, s in enumerate(body) if s.startswith("v_mfma"))
    ws = 0
    for s in body[last + 1:]:
        if _touches(s, acc):
            return None if ws >= 19 else (s, ws)
        ws += _wait_states(s)
    return None


MF = "v_mfma_f32_16x16x32_bf16 a[0:3], v[10:13], v[14:17], a[0:3]"
MFV = "v_mfma_f32_16x16x32_bf16 v[20:23], v[10:13], v[14:17], v[20:23]"


def test_checkers_catch_planted_mistakes():
    # a VALU write of an A operand right before the MFMA, and one wait state
    # after a s_nop 0: caught; two independent instructions between: not
    assert _valu_hazards(["v_mov_b32_e32 v11, v1", MF])
    assert _valu_hazards(["v_mov_b32_e32 v15, v1", "s_nop 0", MF])
    assert not _valu_hazards(["v_mov_b32_e32 v11, v1", "s_nop 1", MF])
    assert not _valu_hazards(["v_mov_b32_e32 v20, v1", MF])
    # a VGPR accumulator written just before the MFMA reads it
    assert _valu_hazards(["v_mov_b32_e32 v21, 0", MFV])
    # an accumulator read 8 wait states after the last MFMA: caught
    assert _unsettled_acc_read([MF, "s_nop 7", "v_accvgpr_read_b32 v0, a0"])
    assert not _unsettled_acc_read([MF, "s_nop 7", "s_nop 7", "s_nop 7",
                                    "v_accvgpr_read_b32 v0, a0"])
    assert _unsettled_acc_read([MFV, "s_nop 7", "v_add_f32_e32 v0, v22, v1"])
    assert not _unsettled_acc_read([MFV, "s_nop 7", "s_nop 7", "s_nop 7",
                                    "v_add_f32_e32 v0, v22, v1"])


def test_no_valu_write_just_before_an_mfma_read(kernels):
    for name, body in kernels.items():
        assert not _valu_hazards(body), (name, _valu_hazards(body)[:3])


def test_loop_keeps_accumulators_in_place(kernels):
    for name, body in kernels.items():
        acc = _acc_regs(body)
        idx = [i for i, s in enumerate(body) if s.startswith("v_mfma")]
        between = body[idx[0]:idx[-1]]
        if any(reg[0] == "a" for reg in acc):
            # AGPR accumulators: no accumulator move at all (in VGPR
            # kernels the compiler may park other values in AGPRs)
            assert not any(s.startswith("v_accvgpr") for s in between), name
        # nor any other access (a copy, spill or reload) of an accumulator
        assert not any(_touches(s, acc) for s in between
                       if not s.startswith("v_mfma")), name
        # tied: every MFMA's result tuple is its accumulator input (AGPRs
        # in the 4-wave GEMM)
        for i in idx:
            ops = _operands(body[i])
            assert ops[0] == ops[3], body[i]
            assert ops[0].startswith("a[") or "skinny" in name, body[i]


def test_results_settle_before_accumulator_reads(kernels):
    for name, body in kernels.items():
        assert _unsettled_acc_read(body) is None, (name, _unsettled_acc_read(body))


def _unsettled_acc_write(body):
    """The last write of an accumulator register before the first MFMA,
    with fewer than 2 wait states between it and the MFMA, or None."""
    acc = _acc_regs(body)
    first = min(i for i, s in enumerate(body) if s.startswith("v_mfma"))
    ws = 0
    for s in reversed(body[:first]):
        ops = _operands(s)
        if s.startswith("v_") and ops and _regs(ops[0]) & acc:
            return None if ws >= 2 else (s, ws)
        ws += _wait_states(s)
    return None


def test_checker_catches_planted_early_write():
    assert _unsettled_acc_write(["v_accvgpr_write_b32 a0, 0", MF])
    assert not _unsettled_acc_write(["v_accvgpr_write_b32 a0, 0", "s_nop 4", MF])
    assert _unsettled_acc_write(["v_mov_b32_e32 v23, 0", MFV])


def test_accumulators_settle_before_the_first_mfma(kernels):
    for name, body in kernels.items():
        assert _unsettled_acc_write(body) is None, (name, _unsettled_acc_write(body))
