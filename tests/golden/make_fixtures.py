"""Writes the reference-held golden vectors used by the sampling tests.

Reads data files shipped with nano-vllm-rs (never its source code):
  benchmarks/attention-validation/native/logits.npz   20 rows x 151936 fp32
      last-position logits of the Qwen3-0.6B validation prompts; every value
      is exactly bf16-representable
  benchmarks/attention-validation/native/eager.json   runs[0].outputs[i].token_ids[0]
      is the token the reference's GPU greedy sampler picked for case i
  benchmarks/results/rust-logits-{0..3}.json          cases 0-3 again, with
      the sampled token in generation.outputs[0].token_ids[0]

Outputs (committed):
  reference_logits.npz  all 20 rows as bf16 bits (row 4 holds an exact tie for
                        the maximum, 16.625 at tokens 9625 and 15344), and
                        expected_greedy for those rows
  reference_greedy.json expected greedy token of all 20 cases plus each case's
                        maximum logit and the indices that attain it

Run in the build container: python tests/golden/make_fixtures.py
"""
import json
import os

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
KEEP_ROWS = list(range(20))


def main() -> None:
    logits = np.load(os.path.join(REF, "benchmarks/attention-validation/native/logits.npz"))
    eager = json.load(open(os.path.join(REF, "benchmarks/attention-validation/native/eager.json")))
    outputs = eager["runs"][0]["outputs"]
    rows = np.stack([logits[str(i)] for i in range(20)]).astype(np.float32)
    bits = rows.view(np.uint32)
    assert int((bits & 0xFFFF).max()) == 0, "logits are expected to be exact bf16 values"
    bf16 = (bits >> 16).astype(np.uint16)
    expected = [int(outputs[i]["token_ids"][0]) for i in range(20)]
    for i in range(4):
        rl = json.load(open(os.path.join(REF, f"benchmarks/results/rust-logits-{i}.json")))
        assert np.array_equal(np.asarray(rl["logits"], np.float32), rows[i])
        assert int(rl["generation"]["outputs"][0]["token_ids"][0]) == expected[i]
    summary = []
    for i in range(20):
        top = float(rows[i].max())
        summary.append({"case": i, "expected_token": expected[i], "max_logit": top,
                        "argmax_indices": [int(j) for j in np.flatnonzero(rows[i] == top)]})
    np.savez_compressed(os.path.join(HERE, "reference_logits.npz"), logits_bf16=bf16[KEEP_ROWS],
                        rows=np.asarray(KEEP_ROWS, np.int32),
                        expected_greedy=np.asarray([expected[i] for i in KEEP_ROWS], np.int32))
    with open(os.path.join(HERE, "reference_greedy.json"), "w") as f:
        json.dump({"source": "benchmarks/attention-validation/native/{logits.npz,eager.json}",
                   "vocab": int(rows.shape[1]), "cases": summary}, f, indent=1)
    print("wrote", len(KEEP_ROWS), "rows;", "expected", expected)


if __name__ == "__main__":
    main()
