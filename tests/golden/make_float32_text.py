"""Writes tests/golden/float32_general_text.json: FP32 values (as bit patterns) and the text
std::to_chars(first, last, value, std::chars_format::general) gives for them with libstdc++
(the form the reference's LSTM params bundle stores its scales in,
operators/quant-lstm/src/lstm/quant_params_io.cc:66-78).  Run from the repository root:
    python tests/golden/make_float32_text.py
Needs g++ (C++17)."""
import json
import subprocess
import tempfile
from pathlib import Path

import numpy as np

SRC = r"""
#include <charconv>
#include <cstdint>
#include <cstdio>
#include <cstring>
int main() {
  unsigned int bits;
  while (std::scanf("%x", &bits) == 1) {
    float v;
    std::memcpy(&v, &bits, 4);
    char buf[64];
    auto r = std::to_chars(buf, buf + 64, v, std::chars_format::general);
    *r.ptr = 0;
    std::printf("%08x %s\n", bits, buf);
  }
}
"""


def values():
    g = np.random.default_rng(20260101)
    out = [np.float32(v) for v in (1e-45, 1.17549435e-38, 3.4028235e38, 1.0, 2.0, 0.5, 1000.0,
                                   65536.0, 1e6, 999999.0, 123456.78, 1234567.0, 1e-4, 1e-5,
                                   9.999999e-05, 0.00012345, 0.1, 0.2, 0.3, 0.0078125,
                                   3.0517578e-05, 1.5258789e-05)]
    for e in range(-40, 39):
        out.append(np.float32(10.0 ** e))
        out.append(np.float32(2.0 ** (e if abs(e) < 127 else 0)))
    exps = g.uniform(-38, 38, 800)
    out += [np.float32(10.0 ** x) for x in exps]
    out += [np.float32(v) for v in g.uniform(0, 1, 200)]
    out += [np.float32(2.0 ** -k) * np.float32(m) for k, m in
            zip(g.integers(0, 40, 100), g.integers(32768, 65536, 100))]
    return [int(np.array(v, np.float32).view(np.uint32)) for v in out if np.isfinite(v) and v > 0]


def main():
    root = Path(__file__).resolve().parent
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = Path(tmp) / "f.cpp", Path(tmp) / "f"
        src.write_text(SRC)
        subprocess.run(["g++", "-std=c++17", "-O1", str(src), "-o", str(exe)], check=True)
        inp = "\n".join(f"{b:08x}" for b in values()) + "\n"
        res = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, check=True)
    pairs = [line.split(" ", 1) for line in res.stdout.splitlines()]
    doc = {"source": "g++ libstdc++ std::to_chars(float, std::chars_format::general)",
           "values": [[b, t] for b, t in pairs]}
    (root / "float32_general_text.json").write_text(json.dumps(doc, indent=0) + "\n")
    print(f"wrote {len(pairs)} values")


if __name__ == "__main__":
    main()
