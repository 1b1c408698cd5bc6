"""Writes tests/golden/decider_cases.json from the reference's own data files (run here, where /root/reference
exists; the output is committed): the fixtures' states and questions (ref/fixtures.json) with the prompts and
answers the reference's CPU run recorded for them (ref/reference_cpu.json): prompt text, option labels, kind,
probabilities and the derived answer (confidence / score / noul). These pin the prompt rendering and the answer
derivation of js/decider.js (web/public/js/prompt.js)."""
import json
import os

REF = "/root/reference/ref"
fx = {f["name"]: f for f in json.load(open(os.path.join(REF, "fixtures.json")))}
out = []
for r in json.load(open(os.path.join(REF, "reference_cpu.json")))["results"]:
    f = fx[r["name"]]
    out.append({"name": r["name"], "state": f["state"], "question": f["question"], "prompt": r["prompt"],
                "kind": r["kind"], "labels": r["slot_labels"], "answer": r["answer"]})
with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "decider_cases.json"), "w") as fh:
    json.dump(out, fh, indent=1, ensure_ascii=False)
print(len(out), "cases")
