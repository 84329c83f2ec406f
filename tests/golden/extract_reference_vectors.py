"""Writes the golden fixtures of this directory from the reference's own unit tests.

The reference keeps two literal known-answer tables for the attention path:

* src/chronos_bolt/model.zig:383-391 -- 281 T5 bucket ids for rel = -140..140 (32 buckets,
  max distance 128), taken there from transformers' `_relative_position_bucket`;
* src/core/attn.zig:191-197 -- the `Mask.pick` truth table.

This script reads those test blocks as text (nothing is compiled or run) and stores the data as
JSON. Run it from the repository root with the reference checkout path:

    python tests/golden/extract_reference_vectors.py /root/reference
"""
import json
import pathlib
import re
import sys


def t5_buckets(src: str) -> list:
    m = re.search(r'test "relativeBucket matches transformers for -140\.\.140".*?\[_\]u8\{([^}]*)\}', src, re.S)
    if not m:
        raise SystemExit("bucket table not found")
    vals = [int(x) for x in m.group(1).replace("\n", " ").split(",") if x.strip()]
    if len(vals) != 281:
        raise SystemExit(f"expected 281 entries, found {len(vals)}")
    return vals


def mask_pick(src: str) -> list:
    m = re.search(r'test "Mask\.pick maps causality.*?\n\}', src, re.S)
    if not m:
        raise SystemExit("Mask.pick test not found")
    rows = []
    for want, c, a, add in re.findall(r"expectEqual\(Mask\.(\w+), Mask\.pick\((\w+), (\w+), (\w+)\)\)", m.group(0)):
        rows.append({"causal": c == "true", "all_keys_valid": a == "true", "additive": add == "true", "mask": want})
    if len(rows) != 5:
        raise SystemExit(f"expected 5 cases, found {len(rows)}")
    return rows


def main() -> None:
    ref = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    out = pathlib.Path(__file__).resolve().parent
    bolt = (ref / "src/chronos_bolt/model.zig").read_text()
    attn = (ref / "src/core/attn.zig").read_text()
    (out / "t5_buckets_32_128.json").write_text(json.dumps({
        "source": "src/chronos_bolt/model.zig:383-391",
        "num_buckets": 32,
        "max_distance": 128,
        "rel_first": -140,
        "buckets": t5_buckets(bolt),
    }) + "\n")
    (out / "mask_pick.json").write_text(json.dumps({
        "source": "src/core/attn.zig:191-197",
        "cases": mask_pick(attn),
    }, indent=1) + "\n")


if __name__ == "__main__":
    main()
