"""Writes tests/golden/decoder_fixtures.json from the decoder fixtures the
nuclis reference holds (data only; nothing of the reference is imported or run).

Source files (MIT, nuclis): inference/src/quant/fixtures/simple.json (Q8_0 row),
k-affine.json (Q4_K and Q5_K rows), k-signed.json (Q6_K row) and iq.json
(IQ4_XS row). They are llama.cpp
7620399f CPU decoder outputs; the reference pins its decoders against them in
inference/src/quant/decode.zig:587-592 and :706-724. Values are stored as the
F32 bit patterns so the fixture is exact.

Run from the repository root: python tests/golden/make_fixtures.py /root/reference
"""
import json
import sys
from pathlib import Path

import numpy as np

WANTED = {"simple.json": (8,), "k-affine.json": (12, 13), "k-signed.json": (14,), "iq.json": (23,)}


def main(reference: str) -> None:
    src = Path(reference) / "inference/src/quant/fixtures"
    rows = []
    revision = None
    for name, encodings in WANTED.items():
        data = json.loads((src / name).read_text())
        revision = data["revision"]
        for row in data["rows"]:
            encoding = row["encoding"]
            if encoding not in encodings:
                continue
            values = np.array([float(v) for v in row["values"]], dtype=np.float32)
            rows.append({
                "source": f"inference/src/quant/fixtures/{name}",
                "encoding": encoding,
                "bytes_hex": bytes(row["bytes"]).hex(),
                "values_f32_hex": values.tobytes().hex(),
            })
    out = Path(__file__).with_name("decoder_fixtures.json")
    out.write_text(json.dumps({"revision": revision, "rows": rows}, indent=1) + "\n")
    print(f"wrote {out} ({len(rows)} rows)")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
