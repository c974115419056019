"""Turns the parity figures a GPU test run recorded (KDEC_PARITY_REPORT, JSON
lines written by tests/conftest.py from model_parity.REPORT) into the
markdown table kept under profiles/.

    KDEC_PARITY_REPORT=parity_report.jsonl \
        python -m pytest tests -m gpu -x -q
    python tests/parity_report.py parity_report.jsonl > profiles/parity_configs.md
"""
from __future__ import annotations

import json
import sys


def fmt(v):
    if v is None:
        return ""
    if isinstance(v, float):
        return f"{v:.3e}"
    return str(v)


def main(path):
    rows = [json.loads(line) for line in open(path) if line.strip()]
    out = ["# GPU parity figures, per configuration",
           "",
           "Every comparison the GPU parity tests make against the oracle (or torch float64 for the single-op",
           "cases), as recorded by one run of the suite on an MI355X:",
           "",
           "```",
           "KDEC_PARITY_REPORT=parity_report.jsonl python -m pytest tests -m gpu -x -q",
           "python tests/parity_report.py parity_report.jsonl > profiles/parity_configs.md",
           "```",
           "",
           "Bars: waveform and forward rel-L2 <= 1e-5, grads rel-L2 <= 1e-4 (a grad that is identically zero",
           "in exact arithmetic, a conv bias in front of an instance norm, is held to an absolute floor and",
           "listed by its max-abs error). `kink` counts the leaky-ReLU inputs (out of `elements`) whose branch",
           "the oracle took from the GPU's input at that site; at each, the oracle's own input lies within",
           "`worst_abs_over_rms` times the site's rms of zero.",
           "",
           "| comparison | rel-L2 | max-abs | notes |",
           "|---|---:|---:|---|"]
    for r in rows:
        extra = {k: v for k, v in r.items() if k not in ("what", "rel_l2", "max_abs")}
        notes = []
        for k, v in extra.items():
            if isinstance(v, dict):
                v = ", ".join(f"{kk} {fmt(vv)}" for kk, vv in v.items())
            notes.append(f"{k}: {fmt(v)}")
        out.append(f"| {r['what']} | {fmt(r['rel_l2'])} | {fmt(r['max_abs'])} | {'; '.join(notes)} |")
    print("\n".join(out))


if __name__ == "__main__":
    main(sys.argv[1])
