"""Register budgets of the chunked grouped GEMMs, from the compiler's
resource report (no GPU needed).

The occupancy these kernels are tuned for is set by their registers as much
as by their LDS:
* the down GEMM (`k_grouped<1, 8, 2, 1, false, *, 48>`) runs two 8-wave blocks
  per CU, four waves per SIMD, so its VGPRs + AGPRs must stay at or below 128
  of the SIMD's 512 per lane (its tall 96-row tiles run one block per CU:
  at most 256);
* the gate/up GEMM with 64-row tiles (`k_grouped<0, 4, 1, 2, false, *, 64>`)
  runs three 4-wave blocks per CU, three waves per SIMD: at most 168 (512 / 3
  in the allocation granule of 8); with the tall 96-row tiles of calls of many
  rows per expert, two blocks per CU: at most 256.
One register over the bound halves the down GEMM's blocks per CU and the
2048-row prefill's down kernel goes from about 106 to 125 us with identical
output bits, which no numerical test sees.

The combine of wide layers (`k_grouped_combine<true>`: a wave per token, its
row indices and scores in SGPRs) keeps every wave of a 2048-token call
resident only at eight waves per SIMD: at most 64 VGPRs and no scratch (at 69
VGPRs it ran 24.6 us instead of 18.0).
"""
import re
import subprocess

import pytest

from veymoe import build

SOURCE = f"{build.CSRC}/grouped.hip"


@pytest.fixture(scope="module")
def kernels(tmp_path_factory):
    """Register counts per kernel of one device-only compile of grouped.hip."""
    return _resources(tmp_path_factory.mktemp("grouped_resources"))


def _resources(tmp_path):
    try:
        hipcc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc is not installed")
    cmd = [hipcc, *build.HIP_FLAGS, "--cuda-device-only", "-Rpass-analysis=kernel-resource-usage",
           "-c", SOURCE, "-o", str(tmp_path / "grouped_device.o")]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    kernels, name = {}, None
    for line in proc.stderr.splitlines():
        m = re.search(r"remark: Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            kernels[name] = {}
            continue
        m = re.search(r"remark: +(VGPRs|AGPRs|ScratchSize \[bytes/lane\]): (\d+)", line)
        if m and name is not None:
            kernels[name][m.group(1)] = int(m.group(2))
    return kernels


def _instances(kernels, prefix):
    found = {k: v for k, v in kernels.items() if prefix in k}
    assert found, f"no kernel matching {prefix} in the resource report"
    return found


def test_grouped_gemm_register_budgets(kernels):
    # template arguments: EPI, waves, column blocks per wave, projections, tail
    # chunk, non-temporal weights, tile rows
    # down: 8 waves, 2 column blocks per wave, 1 projection, no tail chunk;
    # 48-row tiles two blocks per CU, the tall 96-row tiles (88 KB of LDS) one
    for name, r in _instances(kernels, "k_groupedILi1ELi8ELi2ELi1ELb0ELb").items():
        assert name.endswith(("ELi48EEEvNS_13GroupedLaunchE", "ELi96EEEvNS_13GroupedLaunchE")), name
        limit = 256 if name.endswith("ELi96EEEvNS_13GroupedLaunchE") else 128
        assert r["VGPRs"] + r.get("AGPRs", 0) <= limit, (name, r)
    # gate/up: 4 waves, 1 column block per wave, 2 projections, no tail chunk
    for name, r in _instances(kernels, "k_groupedILi0ELi4ELi1ELi2ELb0ELb").items():
        limit = 256 if "ELi96EE" in name else 168
        assert r["VGPRs"] + r.get("AGPRs", 0) <= limit, (name, r)
    assert any("ELi96EE" in name for name in kernels), "the tall gate/up instance"


def test_wave_token_combine_register_budget(kernels):
    for name, r in _instances(kernels, "k_grouped_combineILb1EE").items():
        assert r["VGPRs"] + r.get("AGPRs", 0) <= 64, (name, r)
        assert r.get("ScratchSize [bytes/lane]", 0) == 0, (name, r)
