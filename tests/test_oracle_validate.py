"""Pins the CPU restatement of the value contracts and the host decoding.

The oracle (oracle/validate.py) must report exactly the messages each
planted violation names (tests/contract_cases.py); the host's decoding of a
gs_check_values word must list finiteness messages by tensor, then the value
contracts, in the reference's order.
"""

import pytest

from contract_cases import check_arguments, contract_cases, planted_inputs
from diff_gabor_splatting_amd import _native, rendering
from oracle.validate import value_violations


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_oracle_reports_each_planted_violation(method):
    for label, mutate, expected in contract_cases(method):
        values = planted_inputs(method, mutate)
        assert value_violations(*check_arguments(values, method)) == expected, label


def test_violation_words_decode_in_reference_order():
    names = ["means", "quaternions", "scales"]
    first = _native.CHECK_MAX_TENSORS
    word = (1 << 2) | (1 << 0) | (1 << (first + 0)) | (1 << (first + 10))
    assert rendering.describe_violations(names, word) == [
        "means must contain only finite values",
        "scales must contain only finite values",
        "scales must be strictly positive",
        "frequency_weights must sum to one",
    ]
    assert rendering.describe_violations(names, 0) == []
    every = rendering.describe_violations(names, (1 << (first + 11)) - 1)
    assert every[3:] == list(rendering.VALUE_CONTRACTS)


def test_value_contract_bits_match_the_library_header():
    from pathlib import Path

    header = (Path(__file__).resolve().parents[1] / "include" / "gabor_hip.h").read_text()
    order = ["SCALES_POSITIVE", "OPACITIES_RANGE", "QUATERNIONS_UNIT", "VIEW_LAST_ROW",
             "INTRINSICS_LAST_ROW", "FOCAL_POSITIVE", "ROTATION_ORTHONORMAL",
             "ROTATION_DETERMINANT", "WEIGHTS_NONNEGATIVE", "MAGNITUDES_NONNEGATIVE",
             "WEIGHTS_SUM"]
    assert f"#define GS_CHECK_MAX_TENSORS {_native.CHECK_MAX_TENSORS}" in header
    for k, name in enumerate(order):
        assert f"#define GS_CHECK_{name} (1u << {_native.CHECK_MAX_TENSORS + k})" in header
    assert len(order) == len(rendering.VALUE_CONTRACTS)
