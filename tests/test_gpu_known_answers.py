"""The reference's own known answers, run on the HIP kernels (MI355X)."""

import pytest

from tests._cases import CASE_IDS, CASES, run_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", CASES, ids=CASE_IDS)
def test_known_answer_hip(case, device):
    print(f"[known-answer] {case['id']} ({case['cite']})", flush=True)
    run_case(case, "hip", device)
