"""The 4-wave GEMM issues its MFMAs as inline asm with the accumulator
tied in AGPRs, which the compiler's hazard tracking does not see into.
This compiles the kernels to gfx950 assembly (no GPU needed) and checks,
for every 4-wave GEMM kernel, what that tracking would otherwise
guarantee:
  - no VALU instruction writes an MFMA source register within the
    2 wait states before the MFMA reads it;
  - the main loop moves no accumulator (no v_accvgpr_* between MFMAs);
  - every MFMA result is followed by at least 19 wait states (s_nop) before
    anything outside the MFMAs touches an AGPR."""
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
        if re.match(r"^_Z\S*mot_gemm_kernel\S*Li2E\S*:", raw):
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
    assert found, "no 4-wave GEMM kernels in the assembly"
    return found


def test_every_epilogue_has_a_pinned_kernel(kernels):
    # bf16, SwiGLU, int32 and dequant epilogues, 256 MFMAs each
    assert len(kernels) == 4
    for body in kernels.values():
        assert sum(1 for s in body if s.startswith("v_mfma")) == 256


def _valu_hazards(body):
    """VALU writes of an MFMA source register within 2 wait states of it."""
    bad = []
    for i, s in enumerate(body):
        if not s.startswith("v_mfma"):
            continue
        srcs = set().union(*(_regs(o.strip()) for o in s.split(None, 1)[1].split(",")[1:]))
        ws, k = 0, i - 1
        while k >= 0 and ws < 2:
            p = body[k]
            op = p.split()[0]
            if op.startswith("v_") and not op.startswith("v_mfma"):
                if _regs(p.split(None, 1)[1].split(",")[0].strip()) & srcs:
                    bad.append((p, ws, s))
            ws += _wait_states(p)
            k -= 1
    return bad


def _unsettled_agpr_read(body):
    """The first AGPR access after the last MFMA with fewer than 19 wait
    states between them, or None."""
    last = max(i for i, s in enumerate(body) if s.startswith("v_mfma"))
    ws = 0
    for s in body[last + 1:]:
        if re.search(r"\ba\d+\b|\ba\[", s):
            return None if ws >= 19 else (s, ws)
        ws += _wait_states(s)
    return None


MF = "v_mfma_f32_16x16x32_bf16 a[0:3], v[10:13], v[14:17], a[0:3]"


def test_checkers_catch_planted_mistakes():
    # a VALU write of an A operand right before the MFMA, and one wait state
    # after a s_nop 0: caught; two independent instructions between: not
    assert _valu_hazards(["v_mov_b32_e32 v11, v1", MF])
    assert _valu_hazards(["v_mov_b32_e32 v15, v1", "s_nop 0", MF])
    assert not _valu_hazards(["v_mov_b32_e32 v11, v1", "s_nop 1", MF])
    assert not _valu_hazards(["v_mov_b32_e32 v20, v1", MF])
    # an accumulator read 8 wait states after the last MFMA: caught
    assert _unsettled_agpr_read([MF, "s_nop 7", "v_accvgpr_read_b32 v0, a0"])
    assert not _unsettled_agpr_read([MF, "s_nop 7", "s_nop 7", "s_nop 7",
                                     "v_accvgpr_read_b32 v0, a0"])


def test_no_valu_write_just_before_an_mfma_read(kernels):
    for name, body in kernels.items():
        assert not _valu_hazards(body), (name, _valu_hazards(body)[:3])


def _touches_agpr(s):
    return re.search(r"\ba\d+\b|\ba\[", s) is not None


def test_loop_keeps_accumulators_in_place(kernels):
    for name, body in kernels.items():
        idx = [i for i, s in enumerate(body) if s.startswith("v_mfma")]
        between = body[idx[0]:idx[-1]]
        assert not any(s.startswith("v_accvgpr") for s in between), name
        # nor any other access (a spill or reload) of an AGPR
        assert not any(_touches_agpr(s) for s in between
                       if not s.startswith("v_mfma")), name
        # tied: every MFMA's result tuple is its accumulator input
        for i in idx:
            ops = [o.strip() for o in body[i].split(None, 1)[1].split(",")]
            assert ops[0] == ops[3] and ops[0].startswith("a["), body[i]


def test_results_settle_before_agpr_reads(kernels):
    for name, body in kernels.items():
        assert _unsettled_agpr_read(body) is None, (name, _unsettled_agpr_read(body))


def _unsettled_agpr_write(body):
    """The last AGPR write before the first MFMA, with fewer than 2 wait
    states between it and the MFMA, or None."""
    first = min(i for i, s in enumerate(body) if s.startswith("v_mfma"))
    ws = 0
    for s in reversed(body[:first]):
        op = s.split()[0]
        if _touches_agpr(s) and (op.startswith("v_accvgpr_write") or
                                 op.startswith("v_mov")):
            return None if ws >= 2 else (s, ws)
        ws += _wait_states(s)
    return None


def test_checker_catches_planted_early_write():
    assert _unsettled_agpr_write(["v_accvgpr_write_b32 a0, 0", MF])
    assert not _unsettled_agpr_write(["v_accvgpr_write_b32 a0, 0", "s_nop 4", MF])


def test_accumulators_settle_before_the_first_mfma(kernels):
    for name, body in kernels.items():
        assert _unsettled_agpr_write(body) is None, (name, _unsettled_agpr_write(body))
