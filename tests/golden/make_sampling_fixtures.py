"""Writes sampling_warpers.json: transformers' logits warpers on small rows.

The reference's sampling verification (draft/tree_verification.py:103-106)
warps the target logits with the processor list of prepare_logits_processor
(draft/tree_verification.py:15-32): TemperatureLogitsWarper when
temperature != 1, TopPLogitsWarper when 1e-8 <= top_p < 1, TopKLogitsWarper
when top_k > 0, in that order.  This script applies transformers' own warpers
(the installed transformers, not the reference) row by row to seeded rows and
records the inputs, the warped values and which entries the warpers removed,
so the oracle's restatement (oracle/sampling.py) can be checked against them.

Run: python tests/golden/make_sampling_fixtures.py   (rewrites the JSON beside it)
"""

import json
from pathlib import Path

import numpy as np

import torch
import transformers
from transformers.generation.logits_process import (LogitsProcessorList, TemperatureLogitsWarper,
                                                    TopKLogitsWarper, TopPLogitsWarper)


def processors(temperature, top_p, top_k):
    lst = LogitsProcessorList()
    if temperature >= 1e-5 and temperature != 1.0:
        lst.append(TemperatureLogitsWarper(temperature))
    if 1e-8 <= top_p < 1.0:
        lst.append(TopPLogitsWarper(top_p))
    if top_k > 0:
        lst.append(TopKLogitsWarper(top_k))
    return lst


CASES = [
    # name, dtype, rows, V, sigma, temperature, top_p, top_k, seed
    ("f32_temp_top_p", torch.float32, 4, 128, 2.0, 0.7, 0.9, 0, 1),
    ("f32_temp_top_k", torch.float32, 4, 128, 2.0, 1.3, 1.0, 20, 2),
    ("f32_top_p_top_k", torch.float32, 4, 128, 3.0, 0.8, 0.5, 10, 3),
    ("f32_small_top_p", torch.float32, 4, 128, 1.0, 1.0, 0.05, 0, 4),
    ("f32_top_k_1", torch.float32, 2, 128, 2.0, 1.0, 1.0, 1, 5),
    ("bf16_temp", torch.bfloat16, 2, 128, 3.0, 0.7, 1.0, 0, 6),
    ("f16_temp", torch.float16, 2, 128, 3.0, 1.7, 1.0, 0, 7),
]


def main():
    out = {"source": "transformers " + transformers.__version__ + " TemperatureLogitsWarper / TopPLogitsWarper / "
                     "TopKLogitsWarper, applied per row ([rows, V] input)",
           "cases": []}
    for name, dtype, rows, V, sigma, temp, top_p, top_k, seed in CASES:
        g = torch.Generator().manual_seed(seed)
        x = (torch.randn((rows, V), generator=g) * sigma).to(dtype)
        y = processors(temp, top_p, top_k)(None, x)
        out["cases"].append({
            "name": name, "dtype": {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype],
            "temperature": temp, "top_p": top_p, "top_k": top_k,
            # float32 values in their shortest round-trip form; removed entries as a 0/1 string per row
            "logits": [[float(str(np.float32(v))) for v in r] for r in x.float().numpy()],
            "removed": ["".join(str(int(v)) for v in r) for r in torch.isneginf(y.float())],
            "warped": [[None if np.isneginf(v) else float(str(np.float32(v))) for v in r] for r in y.float().numpy()],
        })
    path = Path(__file__).with_name("sampling_warpers.json")
    path.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
