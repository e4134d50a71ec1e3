"""Writes tests/golden/decoder_reference_results.json from the reference's recorded decoder
results (benchmarks/decoder/results/deep-dive/matrix.json and results/rtx5060ti.json).

Only data is kept: per recorded case its configuration, the executable-plan topology and
temporary-heap statistics with storage reuse off and on, the prompts and the generated tokens.
Run in a container where /root/reference exists: python tests/golden/extract_reference_results.py
"""
import json
from pathlib import Path

SOURCE = Path("/root/reference/benchmarks/decoder/results")
TARGET = Path(__file__).with_name("decoder_reference_results.json")


def main():
    cases = []
    for name in ("deep-dive/matrix.json", "rtx5060ti.json"):
        data = json.loads((SOURCE / name).read_text())
        for index, case in enumerate(data["cases"]):
            plans = {reuse: {key: plan[key] for key in ("nodes", "edges", "temporary_count", "temporary_heap_bytes",
                                                         "topology")}
                     for reuse, plan in case["plans"].items()}
            cases.append(dict(source=name, name=case.get("name", f"case{index}"), config=case["config"], plans=plans,
                              prompts=case["prompts"], generated_tokens=case["generated_tokens"]))
    TARGET.write_text(json.dumps({"cases": cases}, separators=(",", ":")) + "\n")
    print(f"wrote {TARGET} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
