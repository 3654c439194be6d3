"""GGUF inputs for the sanitizer run of the host reader: the hand-assembled
files of test_gguf.py (versions 1-3, alignments, repeated keys, bad UTF-8),
each file cut at every length, and each file with every byte flipped in
turn.  Writes them into the directory given as argv[1]."""
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import struct  # noqa: E402

from test_gguf import hand_file, kv, s64  # noqa: E402


def main(out: str) -> None:
    os.makedirs(out, exist_ok=True)
    bases = {f"v{v}": hand_file(v) for v in (1, 2, 3)}
    bases["align64"] = hand_file(3, align_entry=(4, struct.pack("<I", 64)))
    bases["repeat"] = hand_file(3, extra_kv=kv(b"u8", 4, struct.pack("<I", 7)), extra_kv_count=1)
    bases["utf8"] = struct.pack("<II", 0x46554747, 3) + struct.pack("<QQ", 0, 1) + kv(b"s", 8, s64(b"\xed\xa0\x80\xff"))
    n = 0
    for name, data in bases.items():
        with open(os.path.join(out, f"{name}.gguf"), "wb") as f:
            f.write(data)
        for cut in range(len(data)):
            with open(os.path.join(out, f"{name}_cut{cut}.gguf"), "wb") as f:
                f.write(data[:cut])
        for pos in range(len(data)):
            b = bytearray(data)
            b[pos] ^= 0xFF
            with open(os.path.join(out, f"{name}_flip{pos}.gguf"), "wb") as f:
                f.write(bytes(b))
        n += 1 + 2 * len(data)
    print(f"{n} files in {out}")


if __name__ == "__main__":
    main(sys.argv[1])
