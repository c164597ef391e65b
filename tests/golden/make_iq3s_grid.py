"""Write the IQ3_S grid fixture (tests/golden/iq3s_grid.json).

IQ3_S weights index a fixed 512-entry codebook of four magnitudes (the format's table, llama.cpp's
iq3s_grid, which the reference keeps as `GgufTensorType.iq3sGrid`, Sources/SploshModel/GgufQuant.swift:60).
This script reads that file as text and writes the 512 entries as a JSON fixture; it imports and
runs nothing from the reference. The oracle's and the kernels' copies of the table are checked
against it. Run once where the reference tree is mounted; the output is committed:

    python tests/golden/make_iq3s_grid.py /root/reference
"""
import json
import re
import sys
from pathlib import Path

SOURCE = "Sources/SploshModel/GgufQuant.swift"


def main():
    root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    text = (root / SOURCE).read_text()
    body = re.search(r"static let iq3sGrid: \[UInt32\] = \[(.*?)\]", text, re.S).group(1)
    grid = [int(tok, 16) for tok in re.findall(r"0x[0-9a-fA-F]+", body)]
    assert len(grid) == 512, len(grid)
    dest = Path(__file__).with_name("iq3s_grid.json")
    dest.write_text(json.dumps({"_source": f"{SOURCE}: iq3sGrid (512 entries, byte t = magnitude of element t)",
                                "grid": grid}) + "\n")
    print(f"wrote {dest}")


if __name__ == "__main__":
    main()
