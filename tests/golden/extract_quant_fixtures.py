#!/usr/bin/env python3
"""Copies the Q8_0 / Q5_1 / Q4_0 cases of the reference's dequantizer fixture.

Source: tests/fixtures/quantization.json of the reference (written by its
tools/gen_quant_fixtures.py from the `gguf` package's quantizer and
dequantizer).  Only the three block types the token loop uses are kept, as
data: the GGUF block bytes (base64) and the float32 values gguf decodes them
to.  Run in the build container, where the reference is mounted:

    python3 tests/golden/extract_quant_fixtures.py /root/reference/tests/fixtures/quantization.json
"""
import json
import sys
from pathlib import Path

KEEP = ("Q4_0", "Q5_1", "Q8_0")


def main() -> int:
    src = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/tests/fixtures/quantization.json")
    data = json.loads(src.read_text())
    cases = [c for c in data["cases"] if c["type"] in KEEP]
    out = Path(__file__).with_name("quantization_q.json")
    out.write_text(json.dumps({
        "source": "reference tests/fixtures/quantization.json (gguf quantize/dequantize), Q4_0/Q5_1/Q8_0 cases",
        "cases": cases,
    }, indent=1))
    print(f"wrote {out} ({len(cases)} types)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
