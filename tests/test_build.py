"""Build checks that need no GPU: the step kernel's register budget per launch shape."""
from pathlib import Path

import pytest

from zeno_amd.build import RESOURCES, step_occupancy

REMARKS = """step.hip:1:1: remark: Function Name: _ZN2za12_GLOBAL__N_111step_kernelILi4ELi0ELb0EEEvNS_8StepArgsE
step.hip:1:1: remark:     VGPRs: 238
step.hip:1:1: remark:     Occupancy [waves/SIMD]: 2
step.hip:1:1: remark: Function Name: _ZN2za12_GLOBAL__N_111step_kernelILi1ELi1ELb0EEEvNS_8StepArgsE
step.hip:1:1: remark:     VGPRs: 256
step.hip:1:1: remark:     Occupancy [waves/SIMD]: 1
step.hip:1:1: remark: Function Name: _ZN2za12_GLOBAL__N_111step_kernelILi1ELi2ELb1ELb1EEEvNS_8StepArgsE
step.hip:1:1: remark:     VGPRs: 200
step.hip:1:1: remark:     Occupancy [waves/SIMD]: 2
step.hip:1:1: remark: Function Name: _ZN2za12_GLOBAL__N_111step_kernelILi1ELi0ELb0ELb0EEEvNS_8StepArgsE
step.hip:1:1: remark:     VGPRs: 240
step.hip:1:1: remark:     Occupancy [waves/SIMD]: 2
"""


def test_occupancy_parser():
    assert step_occupancy(REMARKS) == {"4,0,0": 2, "1,1,0": 1, "1,2,1,grouped": 2, "1,0,0": 2}


@pytest.mark.skipif(not Path(RESOURCES).exists(), reason="library not built here")
def test_one_environment_shapes_keep_two_waves_per_simd():
    """Placement 1 without the hash (the rigid pile) and the one-environment LDS shape run
    latency-bound and need two waves per SIMD; above 256 registers the pile's step takes
    2.7x as long."""
    occ = step_occupancy(Path(RESOURCES).read_text())
    assert occ.get("1,1,0") == 2 and occ.get("1,0,0") == 2 and occ.get("1,2,0") == 2, occ


@pytest.mark.skipif(not Path(RESOURCES).exists(), reason="library not built here")
def test_grouped_instances_keep_the_occupancy_of_their_shape():
    """The extended-contact instances (narrow phase grouped by geom-type pair) launch where
    the placement choice scored the ungrouped shape, so they must fit as many waves."""
    occ = step_occupancy(Path(RESOURCES).read_text())
    grouped = [k for k in occ if k.endswith(",grouped")]
    assert len(grouped) == 8, occ  # placements 0-3 with and without the hash
    for k in grouped:
        assert occ[k] >= occ[k[: -len(",grouped")]], (k, occ)
