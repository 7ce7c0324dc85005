"""Write ``known_answers.json``: the reference's known-answer vectors as data.

Every case is transcribed from a numeric assertion in the reference's own tests
(tests/test_roserlhf_losses.py, tests/test_roserlhf_advantages.py) or from a
hand-computed example in its docs, and carries that citation.  Nothing is
imported from the reference; expected values are the literals those files
assert.  Run ``python tests/golden/make_known_answers.py`` to regenerate.

Schema per case: fn (public function name), dtype (tensor dtype for float
args), args (positional tensors as nested lists; bool lists stay bool), kwargs
(keyword arguments; tensors under "tensor_kwargs"), expect (output field ->
value), grad (input name -> expected d(grad_of)/d input), raises.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

LOG2_F32 = float(np.float32(math.log(2.0)))


def case(id, cite, fn, args, *, dtype="float32", kwargs=None, tensor_kwargs=None, expect=None,
         grad=None, grad_of="loss", raises=None, tol=None):
    return {
        "id": id,
        "cite": cite,
        "fn": fn,
        "dtype": dtype,
        "args": args,
        "kwargs": kwargs or {},
        "tensor_kwargs": tensor_kwargs or {},
        "expect": expect or {},
        "grad": grad or {},
        "grad_of": grad_of,
        "raises": raises,
        "tol": tol,
    }


T, F = True, False

CASES = [
    # ---- losses -------------------------------------------------------------
    case("gather_manual", "tests/test_roserlhf_losses.py:18-23", "gather_token_logprobs",
         {"logits": [[[0.0, 1.0], [2.0, -1.0]]], "target_ids": [[1, 0]]},
         expect={"out": [[1.0 - math.log(1.0 + math.e), 2.0 - math.log(math.exp(2.0) + math.exp(-1.0))]]}),
    case("clipped_ratio_one", "tests/test_roserlhf_losses.py:26-35", "clipped_policy_loss",
         {"current_logprobs": [[0.0, 0.0, 0.0]], "old_logprobs": [[0.0, 0.0, 0.0]],
          "advantages": [[1.0, -2.0, 100.0]], "action_mask": [[T, T, F]]},
         expect={"loss": 0.5, "mean_ratio": 1.0, "approximate_kl": 0.0, "clip_fraction": 0.0}),
    case("clipping_sign", "tests/test_roserlhf_losses.py:38-50", "clipped_policy_loss",
         {"current_logprobs": [[LOG2_F32, LOG2_F32]], "old_logprobs": [[0.0, 0.0]],
          "advantages": [[1.0, -1.0]], "action_mask": [[T, T]]},
         expect={"objective": (1.2 - 2.0) / 2, "clip_fraction": 1.0}),
    case("masked_zero_grad", "tests/test_roserlhf_losses.py:53-60", "clipped_policy_loss",
         {"current_logprobs": [[0.0, 0.0, 0.0]], "old_logprobs": [[0.0, 0.0, 0.0]],
          "advantages": [[1.0, 1000.0, -1.0]], "action_mask": [[T, F, T]]},
         grad={"current_logprobs": [[-0.5, 0.0, 0.5]]}),
    case("sequence_log_ratio_mean", "tests/test_roserlhf_losses.py:79-90", "sequence_log_ratio",
         {"current_logprobs": [[0.2, 0.4]], "old_logprobs": [[0.0, 0.0]], "action_mask": [[T, T]]},
         kwargs={"length_normalize": True}, expect={"out": [0.3]}),
    case("sequence_log_ratio_sum", "tests/test_roserlhf_losses.py:79-90", "sequence_log_ratio",
         {"current_logprobs": [[0.2, 0.4]], "old_logprobs": [[0.0, 0.0]], "action_mask": [[T, T]]},
         kwargs={"length_normalize": False}, expect={"out": [0.6]}),
    case("clipped_empty_mask", "tests/test_roserlhf_losses.py:93-98", "clipped_policy_loss",
         {"current_logprobs": [[0.0, 0.0]], "old_logprobs": [[0.0, 0.0]],
          "advantages": [[0.0, 0.0]], "action_mask": [[F, F]]},
         raises={"type": "ValueError", "match": "empty mask"}),
    case("double_sided_strict", "tests/test_roserlhf_losses.py:101-111", "direct_double_sided_mask",
         {"ratios": [0.8, 0.800001, 1.0, 1.199999, 1.2]}, dtype="float64",
         kwargs={"clip_low": 0.2, "clip_high": 0.2}, expect={"out": [F, T, T, T, F]}),
    case("sao_both_tails", "tests/test_roserlhf_losses.py:114-139", "sao_policy_loss",
         {"current_logprobs": [[math.log(0.5), 0.0, math.log(2.0)]],
          "rollout_logprobs": [[0.0, 0.0, 0.0]], "advantages": [[1.0, 1.0, 1.0]],
          "action_mask": [[T, T, T]]}, dtype="float64",
         kwargs={"clip_low": 0.2, "clip_high": 0.2},
         expect={"trusted_mask": [[F, T, F]], "rejected_fraction": 2.0 / 3.0},
         grad={"current_logprobs": [[0.0, -1.0 / 3.0, 0.0]]}),
    case("sao_detached_ratio", "tests/test_roserlhf_losses.py:142-159", "sao_policy_loss",
         {"current_logprobs": [[-0.5]], "rollout_logprobs": [[-0.6]], "advantages": [[2.0]],
          "action_mask": [[T]]}, dtype="float64",
         kwargs={"clip_low": 0.2, "clip_high": 0.2, "detach_ratio": True},
         grad={"current_logprobs": [[-2.0 * math.exp(0.1)]], "rollout_logprobs": None}),
    case("sao_attached_ratio", "tests/test_roserlhf_losses.py:161-174", "sao_policy_loss",
         {"current_logprobs": [[-0.5]], "rollout_logprobs": [[-0.6]], "advantages": [[2.0]],
          "action_mask": [[T]]}, dtype="float64",
         kwargs={"clip_low": 0.2, "clip_high": 0.2, "detach_ratio": False},
         grad={"current_logprobs": [[-2.0 * math.exp(0.1) * (1.0 - 0.5)]],
               "rollout_logprobs": None}),
    case("sao_masks_observations", "tests/test_roserlhf_losses.py:177-195", "sao_policy_loss",
         {"current_logprobs": [[0.0, 0.0, 0.0]], "rollout_logprobs": [[0.0, -10.0, 0.0]],
          "advantages": [[1.0, 1000.0, -1.0]], "action_mask": [[T, F, T]]},
         kwargs={"clip_low": 0.2, "clip_high": 0.2},
         expect={"rejected_fraction": 0.0, "trusted_mask": [[T, F, T]]},
         grad={"current_logprobs": [[-0.5, 0.0, 0.5]]}),
    case("evidence_no_grad", "tests/test_roserlhf_losses.py:198-211", "clipped_policy_loss",
         {"current_logprobs": [[0.0, 0.0]], "old_logprobs": [[0.0, 0.0]],
          "advantages": [[1.0, 1.0]], "action_mask": [[T, T]]},
         grad={"current_logprobs": [[-0.5, -0.5]], "old_logprobs": None, "advantages": None}),
    case("gspo_geometric_mean", "tests/test_roserlhf_losses.py:214-236", "gspo_policy_loss",
         {"current_logprobs": [[math.log(4.0), 0.0], [0.0, 999.0]],
          "rollout_logprobs": [[0.0, 0.0], [0.0, 0.0]], "sequence_advantages": [1.0, 1.0],
          "action_mask": [[T, T], [T, F]]}, dtype="float64",
         kwargs={"clip_low": 0.5, "clip_high": 2.0},
         expect={"sequence_ratios": [2.0, 1.0], "objective": 1.5},
         grad={"current_logprobs": [[-0.5, -0.5], [-0.5, 0.0]]}),
    case("gspo_token_distinct", "tests/test_roserlhf_losses.py:271-286", "gspo_token_policy_loss",
         {"current_logprobs": [[0.0, 0.0]], "rollout_logprobs": [[0.0, 0.0]],
          "token_advantages": [[1.0, -2.0]], "action_mask": [[T, T]]}, dtype="float64",
         kwargs={"clip_low": 0.2, "clip_high": 0.2},
         grad={"current_logprobs": [[-0.5, 1.0]]}),
    case("sapo_gate_on_policy", "tests/test_roserlhf_losses.py:289-305", "sapo_policy_loss",
         {"current_logprobs": [[0.0, 0.0]], "rollout_logprobs": [[0.0, 0.0]],
          "token_advantages": [[2.0, -3.0]], "action_mask": [[T, T]]}, dtype="float64",
         kwargs={"tau_positive": 1.0, "tau_negative": 5.0},
         expect={"mean_gradient_gate": 1.0},
         grad={"current_logprobs": [[-1.0, 1.5]]}),
    case("docs_one_batch", "docs/agentic-rl/derivations-and-code.md:1119-1156", "clipped_policy_loss",
         {"current_logprobs": [[-0.9, -0.6], [-0.1, -1.0]],
          "old_logprobs": [[-1.0, -0.5], [-0.2, -0.7]],
          "advantages": [[1.0, 1.0], [-0.5, -0.5]], "action_mask": [[1, 1], [1, 0]]},
         kwargs={"clip_low": 0.2}, expect={"loss": -0.48581}, tol=5e-6),
    # ---- advantages ---------------------------------------------------------
    case("returns_cut_terminal", "tests/test_roserlhf_advantages.py:14-18", "discounted_returns",
         {"rewards": [[1.0, 2.0, 100.0]]}, kwargs={"gamma": 0.5},
         tensor_kwargs={"terminated": [[F, T, F]]}, expect={"out": [[2.0, 2.0, 100.0]]}),
    case("returns_bootstrap", "tests/test_roserlhf_advantages.py:21-29", "discounted_returns",
         {"rewards": [[1.0, 2.0]]}, kwargs={"gamma": 0.5},
         tensor_kwargs={"terminated": [[F, F]], "bootstrap_value": [10.0]},
         expect={"out": [[4.5, 7.0]]}),
    case("returns_skip_padding", "tests/test_roserlhf_advantages.py:32-36", "discounted_returns",
         {"rewards": [[1.0, 2.0, 999.0]]}, tensor_kwargs={"valid_mask": [[T, T, F]]},
         expect={"out": [[3.0, 2.0, 0.0]]}),
    case("gae_lambda_one", "tests/test_roserlhf_advantages.py:39-52",
         "generalized_advantage_estimation",
         {"rewards": [[1.0, 2.0, 3.0]], "values": [[0.5, 0.7, 1.1]]},
         kwargs={"gamma": 0.9, "gae_lambda": 1.0}, tensor_kwargs={"terminated": [[F, F, T]]},
         expect={"out0": [[5.23 - 0.5, 4.7 - 0.7, 3.0 - 1.1]], "out1": [[5.23, 4.7, 3.0]]}),
    case("leave_one_out", "tests/test_roserlhf_advantages.py:55-59", "leave_one_out_advantages",
         {"rewards": [[0.0, 1.0, 2.0]]}, expect={"out": [[-1.5, 0.0, 1.5]]}),
    case("leave_one_out_singleton", "tests/test_roserlhf_advantages.py:62-64",
         "leave_one_out_advantages", {"rewards": [[1.0]]},
         raises={"type": "ValueError", "match": "group_size"}),
    case("group_uniform_zero", "tests/test_roserlhf_advantages.py:67-71",
         "group_standardized_advantages", {"rewards": [[1.0] * 4, [1.0] * 4]},
         expect={"out": [[0.0] * 4, [0.0] * 4]}, tol=0.0),
    case("group_mean0_std1", "tests/test_roserlhf_advantages.py:74-80",
         "group_standardized_advantages", {"rewards": [[0.0, 1.0, 2.0, 3.0]]},
         expect={"out": [[-1.5 / math.sqrt(1.25), -0.5 / math.sqrt(1.25), 0.5 / math.sqrt(1.25),
                          1.5 / math.sqrt(1.25)]]}),
    case("broadcast_turns", "tests/test_roserlhf_advantages.py:83-88",
         "broadcast_turn_advantages",
         {"turn_advantages": [[2.0, -1.0]], "turn_ids": [[0, 0, 0, 1, 1]],
          "action_mask": [[T, F, T, F, T]]}, expect={"out": [[2.0, 0.0, 2.0, 0.0, -1.0]]}, tol=0.0),
    case("broadcast_invalid_turn", "tests/test_roserlhf_advantages.py:91-97",
         "broadcast_turn_advantages",
         {"turn_advantages": [[1.0]], "turn_ids": [[2]], "action_mask": [[T]]},
         raises={"type": "ValueError", "match": "invalid turn"}),
    case("skip_obs_bridges", "tests/test_roserlhf_advantages.py:100-110",
         "skip_observation_generalized_advantage_estimation",
         {"rewards": [[0.0, 1.0]], "action_end_values": [[0.2, 0.4]],
          "next_action_values": [[0.4, 0.0]]}, kwargs={"gamma": 1.0, "gae_lambda": 1.0},
         tensor_kwargs={"terminated": [[F, T]]},
         expect={"out0": [[0.8, 0.6]], "out1": [[1.0, 1.0]]}),
    case("skip_obs_terminal", "tests/test_roserlhf_advantages.py:113-121",
         "skip_observation_generalized_advantage_estimation",
         {"rewards": [[1.0]], "action_end_values": [[0.25]], "next_action_values": [[999.0]]},
         tensor_kwargs={"terminated": [[T]]}, expect={"out0": [[0.75]], "out1": [[1.0]]}),
    case("skip_obs_bootstrap", "tests/test_roserlhf_advantages.py:124-133",
         "skip_observation_generalized_advantage_estimation",
         {"rewards": [[2.0]], "action_end_values": [[1.0]], "next_action_values": [[5.0]]},
         kwargs={"gamma": 0.5}, tensor_kwargs={"terminated": [[F]]},
         expect={"out0": [[3.5]], "out1": [[4.5]]}),
    case("skip_obs_padding", "tests/test_roserlhf_advantages.py:136-145",
         "skip_observation_generalized_advantage_estimation",
         {"rewards": [[1.0, 999.0, 2.0]], "action_end_values": [[0.0, 0.0, 0.0]],
          "next_action_values": [[0.0, 0.0, 0.0]]},
         tensor_kwargs={"terminated": [[F, F, T]], "valid_mask": [[T, F, T]]},
         expect={"out0": [[3.0, 0.0, 2.0]], "out1": [[3.0, 0.0, 2.0]]}),
    case("skip_obs_lambda_zero", "tests/test_roserlhf_advantages.py:148-156",
         "skip_observation_generalized_advantage_estimation",
         {"rewards": [[0.0, 1.0]], "action_end_values": [[0.2, 0.4]],
          "next_action_values": [[0.4, 0.0]]}, kwargs={"gae_lambda": 0.0},
         tensor_kwargs={"terminated": [[F, T]]}, expect={"out0": [[0.2, 0.6]]}),
    case("returns_docs_bootstrap", "docs/agentic-rl/source-lab.md:223-228", "discounted_returns",
         {"rewards": [[1.0, 2.0]]}, kwargs={"gamma": 0.5},
         tensor_kwargs={"bootstrap_value": [10.0]}, expect={"out": [[4.5, 7.0]]}),
    case("loo_docs", "docs/agentic-rl/derivations-and-code.md:208-220",
         "leave_one_out_advantages", {"rewards": [[0.0, 1.0, 2.0]]},
         expect={"out": [[-1.5, 0.0, 1.5]]}),
]


def main() -> None:
    out = Path(__file__).with_name("known_answers.json")
    out.write_text(json.dumps({"source": "chtho-like/rosellm tests and docs (transcribed)",
                               "cases": CASES}, indent=1))
    print(f"wrote {len(CASES)} cases to {out}")


if __name__ == "__main__":
    main()
