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
    "loss_contract_global_mean": {
        "source": "tests/test_global_loss_and_clock.py:127-152",
        "microbatches": [
            {"losses": [1.0, 2.0, 3.0], "mask": [1.0, 0.0, 1.0]},
            {"losses": [4.0, 5.0], "mask": [1.0, 0.0]},
        ],
        "nominal_global_loss_scale": 8.0,
        "expected_local_loss_sum": [4.0, 4.0],
        "expected_local_loss_weight": [2.0, 1.0],
        "expected_normalized_grads": [[1 / 3, 0.0, 1 / 3], [1 / 3, 0.0]],
    },
    "loss_aggregation": {
        "source": "tests/test_global_loss_and_clock.py:241-253",
        "outputs": [[2.0, 1.0], [6.0, 1.0], [12.0, 2.0]],
        "expected_numerator": 20.0,
        "expected_weight": 4.0,
        "expected_mean": 5.0,
    },
    "training_clock": {
        "source": "tests/test_global_loss_and_clock.py:207-219",
        "total_gbs": 10,
        "global_data_cursor": 20,
        "successful_optimizer_steps": 3,
        "attempts": [False, True],
        "expected_returns": [0, 10],
        "expected_cursor": 40,
        "expected_steps": 4,
    },
    "training_clock_restore": {
        "source": "tests/test_global_loss_and_clock.py:221-239",
        "checkpoint": {"consumed_train_samples": 12, "global_data_cursor": 30, "successful_optimizer_steps": 4},
        "legacy_checkpoint": {"consumed_train_samples": 12},
        "iteration": 7,
        "expected": [30, 4],
        "expected_legacy": [12, 7],
    },
    "sample_slots": {
        "source": "tests/test_global_loss_and_clock.py:160-200 (the slots listed here follow from its sequences)",
        "mbs_sequences": [[[4, 8], [2, 8]], [[2, 8], [2, 8]]],
        "pipeline_sample_offsets": [0, 6],
        "total_gbs": 10,
        "cases": [
            [[0, 0, 1, 0, 0], [0, 1, 2, 3]],
            [[0, 0, 2, 0, 0], [0, 1]],
            [[0, 0, 2, 1, 0], [2, 3]],
            [[0, 1, 2, 1, 0], [5]],
            [[1, 0, 2, 1, 0], [7]],
            [[1, 1, 1, 0, 0], [8, 9]],
            [[0, 0, 1, 0, 10], [10, 11, 12, 13]],
        ],
    },
    "synthetic_gpt_batch": {
        "source": "grad_sync/loss.py:100-119 (values computed by hand from the LCG); "
                  "tests/test_global_loss_and_clock.py:202-205 uses the (0,1)/(2,3), s 4, V 100 batches",
        "cases": [
            {"ids": [0, 1], "seq": 4, "vocab": 100, "tokens": [[0, 45, 90, 35], [45, 90, 35, 80]],
             "mask": [[0, 1, 1, 1], [1, 1, 1, 0]]},
            {"ids": [2, 3], "seq": 4, "vocab": 100, "tokens": [[90, 35, 80, 25], [35, 80, 25, 70]],
             "mask": [[1, 1, 0, 1], [1, 0, 1, 1]]},
            {"ids": [3, 8], "seq": 6, "vocab": 50257,
             "tokens": [[16631, 28976, 41321, 3409, 15754, 28099], [27597, 39942, 2030, 14375, 26720, 39065]],
             "mask": [[1, 0, 1, 1, 1, 0], [0, 1, 1, 1, 0, 1]]},
        ],
    },
    "dynamic_loss_scale": {
        "source": "optimizer/grad_scaler.py:99-119 (update rule), arguments.py:644 (hysteresis 2)",
        "initial_scale": 65536.0,
        "min_scale": 16384.0,
        "growth_factor": 2.0,
        "backoff_factor": 0.5,
        "growth_interval": 3,
        "hysteresis": 2,
        "found_inf": [False, False, False, True, False, True, True, True, True, False, False, False],
        "expected_scale": [65536.0, 65536.0, 131072.0, 131072.0, 131072.0, 65536.0, 32768.0, 16384.0, 16384.0,
                           16384.0, 16384.0, 32768.0],
    },
    "runtime_evidence_four_to_two": {
        "source": "tests/test_gradient_executor.py:70-148",
        "groups": [["pg-a", [0]], ["pg-b", [0]]],
        "fragments": [["f0", "p0", "pg-a", 2, 0], ["f1", "p1", "pg-b", 2, 1], ["f2", "p2", "pg-a", 2, 2],
                      ["f3", "p3", "pg-b", 2, 3]],
        "tensors": {"p0": [1.0, 2.0], "p1": [2.0, 3.0], "p2": [3.0, 4.0], "p3": [4.0, 5.0]},
        "cap_bytes": 1024,
        "iterations": 2,
        "expected_collectives": {"tensor": 4, "block": 2},
        "expected_payload_bytes": 32,
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
