"""Writes tests/golden/pplx_answers.json: the answer-step vectors that the
reference's own test data holds.

Sources (data only, read as JSON text; nothing of the reference is run):
  tests/fixtures/pplx_flash/reference.json  -- per case, the request's
      questions, the readout logits per question key and the response's
      answers (written by the reference's Python protocol implementation).
  src/models/pplx_flash/input.rs:327-349    -- the known answers of its
      json_text and options tests, restated here as data.

The checkpoint's temperature (decision_config.json) is not in the reference.
Every logit pair fixes it through p_i/p_j = exp((l_i - l_j)/T); the fixture
records the median over all pairs, and the answer test then checks every
probability, choice, score and confidence against the response with the
reference's own tolerance (1e-4, pplx_flash/mod.rs compare()).

Usage: python tests/golden/make_pplx_answers.py [/root/reference]
"""
import json
import math
import statistics
import sys
from pathlib import Path

ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
data = json.loads((ref / "tests/fixtures/pplx_flash/reference.json").read_text())

cases, ratios = [], []
for case in data["cases"]:
    questions = case["request"]["questions"]
    answers = case["response"]["answers"]
    for key, logits in case["logits"].items():
        a = answers[key]
        p = [1 - a["noul"], a["noul"]] if a["type"] == "noul" else list(a["probabilities"].values())
        for i in range(1, len(logits)):
            ratios.append((logits[i] - logits[0]) / math.log(p[i] / p[0]))
    cases.append({"questions": questions, "keys": case["keys"], "counts": case["counts"],
                  "logits": case["logits"], "answers": answers, "usage": case["response"]["usage"]})

out = {
    "_source": "tests/fixtures/pplx_flash/reference.json and src/models/pplx_flash/input.rs:327-349 (data only)",
    "temperature_fit": statistics.median(ratios),
    "temperature_fit_spread": max(ratios) - min(ratios),
    "tolerance": 1e-4,
    "cases": cases,
    "json_text": [{
        "value": {"small": 1e-7, "large": 1e16, "negative_zero": -0.0, "unicode": ["中文", True, None]},
        "text": "{\"small\": 1e-07, \"large\": 1e+16, \"negative_zero\": -0.0, \"unicode\": [\"中文\", true, null]}",
    }],
    "options": [
        {"question": {"type": "choice", "criteria": {"z": None, "a": {"name": "value"}}},
         "keys": ["z", "a"], "legend": ["z", "a: {\"name\": \"value\"}"]},
        {"question": {"type": "noul", "criteria": {"true": "", "false": "negative"}},
         "keys": ["false", "true"], "legend": ["negative", "Yes / true"]},
        {"question": {"type": "score", "criteria": ["one"]}, "error": "score requires at least two levels"},
    ],
}
dst = Path(__file__).with_name("pplx_answers.json")
dst.write_text(json.dumps(out, indent=1, ensure_ascii=False) + "\n")
print(dst, "temperature", out["temperature_fit"], "spread", out["temperature_fit_spread"])
