#!/usr/bin/env python3
"""Extracts the known-answer examples of the Gyro format specification into spec_kat.json.

Reads third_party/agention-gyro/SPEC.md section 10 (lines 337-436 of the reference tree) as
text: the example block bytes, the scale, and every printed table row (step, state,
state & 0x7fff, codebook indices and the decoded values rounded to 6 decimals). Run in a
container where the reference tree is mounted; the output JSON is the committed fixture.
"""
import json
import re
import sys
from pathlib import Path

SPEC = Path(sys.argv[1] if len(sys.argv) > 1 else
            "/root/reference/third_party/agention-gyro/SPEC.md")
OUT = Path(__file__).resolve().parent / "spec_kat.json"


def hexbytes(text):
    return [int(b, 16) for b in re.findall(r"\b[0-9a-f]{2}\b", text)]


def main():
    lines = SPEC.read_text().splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith("## 10. Worked example"))
    end = next(i for i, l in enumerate(lines) if l.startswith("## 11."))
    sec = lines[start:end]
    cases = []
    cur = None
    i = 0
    while i < len(sec):
        l = sec[i]
        m = re.match(r"### 10\.(\d) (\S+) block, d = (-?[0-9.]+)", l)
        if m:
            cur = {"section": f"10.{m.group(1)}", "type": m.group(2), "d": float(m.group(3)),
                   "bytes": [], "rows": []}
            cases.append(cur)
        elif cur is not None and l.startswith("bytes:"):
            blob = l[len("bytes:"):]
            j = i + 1
            while j < len(sec) and sec[j].startswith("   ") and not sec[j].strip().startswith("\\"):
                blob += " " + sec[j]
                j += 1
            blob = blob.replace("|", " ")
            cur["bytes"] = hexbytes(blob.split("\\")[0] if "\\" in blob else blob)
        elif cur is not None:
            r = re.match(r"^\s+(\d+)\s+0x([0-9a-f]{4})\s+0x([0-9a-f]{4})\s+(\d+)\s+(.*)$", l)
            if r:
                rest = r.group(5).split()
                row = {"t": int(r.group(1)), "state": int(r.group(2), 16),
                       "masked": int(r.group(3), 16), "idx0": int(r.group(4))}
                if cur["type"] == "TQP5":
                    row["w"] = [float(v) for v in rest]
                else:
                    row["idx1"] = int(rest[0])
                    row["w"] = [float(v) for v in rest[1:]]
                cur["rows"].append(row)
        i += 1
    ids = {"TQK4": 151, "TQ2_T": 144, "TQP5": 147}
    for c in cases:
        c["type_id"] = ids[c["type"]]
    OUT.write_text(json.dumps({"source": "third_party/agention-gyro/SPEC.md section 10",
                               "cases": cases}, indent=1) + "\n")
    print(OUT, [(c["type"], len(c["bytes"]), len(c["rows"])) for c in cases])


if __name__ == "__main__":
    main()
