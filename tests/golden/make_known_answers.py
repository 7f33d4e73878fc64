"""Write tests/golden/known_answers.json: the known-answer vectors of the
reference's own tests for the hot path, transcribed as data (inputs and
expected outputs).  Nothing here runs reference code; each record cites the
test it comes from.

    python tests/golden/make_known_answers.py
"""

import json
from pathlib import Path

RECORDS = {
    "executor_strided_pack": {
        "source": "tests/test_gradient_executor.py:311-361",
        "main_grad_shape": [4, 3],
        "main_grad": list(range(12)),
        "partition_dim": 0,
        "fragments": [
            {"id": "f-even", "order": 0, "numel": 6, "segments": [[0, 1], [2, 1]]},
            {"id": "f-odd", "order": 1, "numel": 6, "segments": [[1, 1], [3, 1]]},
        ],
        "cap_bytes": 1024,
        "mode": "block",
        "all_reduce": "mul2",
        "normalization_scale": 0.5,
        "expected_packed": [[0, 1, 2, 6, 7, 8, 3, 4, 5, 9, 10, 11]],
        "expected_main_grad": list(range(12)),
    },
    "executor_scratch_tail": {
        "source": "tests/test_gradient_executor.py:397-439",
        "tensors": {"large-param": list(range(8)), "small-param": [10, 11, 12, 13]},
        "mode": "tensor",
        "all_reduce": "add100",
        "iterations": 2,
        "expected_numels": [8, 4, 8, 4],
        "expected_scratch_tail": [104, 105, 106, 107],
    },
    "executor_replicated_half": {
        "source": "tests/test_gradient_executor.py:363-395",
        "dtype": "float16",
        "main_grad": [1, 2, 3, 4],
        "contribution_scale": 0.5,
        "all_reduce": "mul2",
        "expected_main_grad": [1, 2, 3, 4],
    },
    "bucket_plan_tensor_vs_block": {
        "source": "tests/test_gradient_bucket_plan.py:58-77",
        "fragments": [[0, "pg-a", "float32", 8], [1, "pg-b", "float32", 8], [2, "pg-a", "float32", 8], [3, "pg-b", "float32", 8]],
        "groups": [["pg-a", [0, 1]], ["pg-b", [0, 2]]],
        "cap_bytes": 33554432,
        "expected_tensor_buckets": 4,
        "expected_block_buckets": 2,
    },
    "bucket_plan_boundaries": {
        "source": "tests/test_gradient_bucket_plan.py:79-106",
        "fragments": [[0, "pg-a", "float16", 4], [1, "pg-a", "float32", 4], [2, "pg-b", "float32", 4], [3, "pg-b", "float32", 20]],
        "groups": [["pg-a", [0, 1]], ["pg-b", [0, 2]]],
        "cap_bytes": 16,
        "expected_block_buckets": 4,
        "expected_last_oversized": True,
        "expected_last_numel": 20,
    },
    "canonical_clip": {
        "source": "tests/test_optimizer_semantics.py:454-538",
        "owned_grads": [[3.0, 4.0, 0.0, 0.0]],
        "max_norm": 2.0,
        "expected_norm": 5.0,
        "expected_clipped": [[1.2, 1.6, 0.0, 0.0]],
        "expected_zeros": 2.0,
        "expected_inf_norm": 1.6,
    },
    "adamw_step1": {
        "source": "tests/test_gpt_numerical_evidence.py:469-504",
        "param": [1.0, -2.0],
        "grad": [3.0, 4.0],
        "max_norm": 1.0,
        "lr": 0.01,
        "betas": [0.9, 0.95],
        "eps": 1e-8,
        "weight_decay": 0.1,
        "expected_norm": 5.0,
        "expected_coefficient_formula": "1/(5+1e-6)",
        "expected_exp_avg_over_grad": 0.1,
        "expected_exp_avg_sq_over_grad_sq": 0.05,
    },
    "main_grad_accumulation": {
        "source": "tests/test_local_ddp_runtime.py:48-72",
        "param": [1.0, 2.0],
        "inputs": [[2.0, 4.0], [1.0, 1.0]],
        "expected_main_grad_after": [[2.0, 4.0], [3.0, 5.0]],
        "expected_unused_main_grad": [0.0],
    },
}


def main():
    out = Path(__file__).with_name("known_answers.json")
    out.write_text(json.dumps(RECORDS, indent=1, sort_keys=True) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
