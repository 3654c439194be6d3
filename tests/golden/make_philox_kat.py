"""Extract the Philox-4x32-10 known-answer vectors that fuel's own tests hold
(fuel-cpu-kernels/src/philox_kat.rs:18-75, the Random123 kat_vectors) into
philox4x32_10_kat.json.  Run in the build container, where /root/reference
exists; the JSON is the committed fixture (data only)."""
import json
import os
import re
import sys

SRC = "/root/reference/fuel-cpu-kernels/src/philox_kat.rs"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "philox4x32_10_kat.json")


def main() -> int:
    text = open(SRC).read()
    row = re.compile(
        r"\(\[(0x[0-9a-f]+), (0x[0-9a-f]+), (0x[0-9a-f]+), (0x[0-9a-f]+)\], "
        r"\[(0x[0-9a-f]+), (0x[0-9a-f]+)\], "
        r"\[(0x[0-9a-f]+), (0x[0-9a-f]+), (0x[0-9a-f]+), (0x[0-9a-f]+)\]\)"
    )
    vecs = []
    for m in row.finditer(text):
        v = [int(g, 16) for g in m.groups()]
        vecs.append({"ctr": v[0:4], "key": v[4:6], "out": v[6:10]})
    json.dump({"source": "fuel-cpu-kernels/src/philox_kat.rs (Random123 kat_vectors)",
               "vectors": vecs}, open(OUT, "w"), indent=0)
    print(f"{len(vecs)} vectors -> {OUT}")
    return 0 if vecs else 1


if __name__ == "__main__":
    sys.exit(main())
