"""Write the GGUF golden-block fixtures (tests/golden/gguf_golden_blocks.json).

The reference's test suite holds one real block of each quantised GGUF format together with the
float32 values its decoder produces for it (Tests/SploshOracleTests/GgufGoldenBlocks.swift:22-330, one block of each of
the eight formats). This script reads that file as text and copies the bytes and
values into a JSON fixture; it imports and runs nothing from the reference. It is run once, in a
container where the reference tree is mounted, and its output is committed:

    python tests/golden/make_gguf_golden.py /root/reference
"""
import json
import re
import sys
from pathlib import Path

SOURCE = "Tests/SploshOracleTests/GgufGoldenBlocks.swift"


def parse(text):
    blocks = {}
    pattern = re.compile(
        r"static let (\w+) = GgufGoldenBlock\(\s*type:\s*\.(\w+),\s*tensor:\s*\"([^\"]+)\",\s*"
        r"bytes:\s*\[(.*?)\],\s*values:\s*\[(.*?)\]\)",
        re.S)
    for name, kind, tensor, raw_bytes, raw_values in pattern.findall(text):
        data = [int(tok, 16) for tok in re.findall(r"0x[0-9a-fA-F]+", raw_bytes)]
        values = [tok for tok in re.findall(r"[-+]?\d+\.?\d*(?:[eE][-+]?\d+)?", raw_values)]
        blocks[name] = {"type": kind, "tensor": tensor, "bytes": data, "values": values}
    return blocks


def main():
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    blocks = parse((root / SOURCE).read_text())
    expected = {"q4K": 144, "q5K": 176, "q6K": 210, "q3K": 110, "q8_0": 34, "iq4NL": 18, "iq4XS": 136, "iq3S": 110}
    out = {}
    for name, size in expected.items():
        block = blocks[name]
        assert len(block["bytes"]) == size, (name, len(block["bytes"]))
        assert len(block["values"]) == (32 if size in (34, 18) else 256), (name, len(block["values"]))
        out[name] = block
    out["_source"] = f"{SOURCE} (one block of each of the eight formats); values are float32 printed with 9 digits"
    dest = Path(__file__).with_name("gguf_golden_blocks.json")
    dest.write_text(json.dumps(out) + "\n")
    print(f"wrote {dest}")


if __name__ == "__main__":
    main()
