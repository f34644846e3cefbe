"""The prefill GEMM's inline-assembly weight loads, checked on its gfx950 assembly (CPU):
no instruction touches a register whose load may still be outstanding.  A register
handed to another value while such a load is in flight is overwritten when the load
returns (an address register corrupted that way made the GPU fault)."""

import shutil
import subprocess
from pathlib import Path

import pytest

from isa_inflight import inflight_hazards, kernel_names

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "vllm-neuron_amd" / "csrc" / "expert_prefill.hip"


@pytest.fixture(scope="module")
def prefill_asm(tmp_path_factory):
    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "expert_prefill.s"
    subprocess.run([hipcc, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                    "-target-feature", "-Xclang", "-packed-fp32-ops", "-S",
                    "--cuda-device-only", str(SRC), "-o", str(out)],
                   check=True, capture_output=True, timeout=600)
    return out.read_text()


def test_prefill_asm_loads_not_touched_in_flight(prefill_asm):
    names = kernel_names(prefill_asm, "_ZN5mxmoe19prefill_gemm_kernel")
    assert len(names) == 4, names  # gate_up and down, MXFP4 and MXFP8
    for name in names:
        hazards = inflight_hazards(prefill_asm, name)
        assert not hazards, f"{name}: {hazards[:5]}"


def test_checker_finds_a_planted_hazard():
    """A register reused after an asm load and before its wait is reported."""
    asm = "\n".join([
        "k:", "\t;;#ASMSTART", "\tglobal_load_dwordx4 v[4:7], v[0:1], off", "\t;;#ASMEND",
        "\tv_mov_b32_e32 v5, 0", "\ts_waitcnt vmcnt(0)", "\tv_mov_b32_e32 v6, 1",
        "\ts_endpgm", ".Lfunc_end0:"])
    hazards = inflight_hazards(asm, "k")
    assert [h[1] for h in hazards] == [[5]]
