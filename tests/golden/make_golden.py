"""Writes tests/golden/mt19937_libstdcxx.json: raw outputs of libstdc++'s
std::mt19937, the generator the reference's test inputs are drawn from
(src/tests/tilemix_test.cu:47, seed m*131 + n*17 + d).

The C++ program below is compiled with the system g++ and run once; its output
is the fixture. Seeds: the C++ standard's default seed 5489, and the seeds of
the reference test shapes used by this repository's tests.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import subprocess
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
SHAPES = [(17, 65, 1), (17, 129, 1), (129, 65, 17), (137, 73, 31), (129, 131, 17), (64, 64, 64),
          (33, 47, 8), (1, 1, 1)]
PREFIX = 256

PROGRAM = r"""
#include <cstdio>
#include <cstdlib>
#include <random>
int main(int argc, char** argv) {
    for (int i = 1; i < argc; ++i) {
        const unsigned long seed = std::strtoul(argv[i], nullptr, 10);
        std::mt19937 g(static_cast<std::mt19937::result_type>(seed));
        std::printf("%lu", seed);
        for (int k = 0; k < %PREFIX%; ++k) std::printf(" %u", static_cast<unsigned>(g()));
        std::mt19937 h(static_cast<std::mt19937::result_type>(seed));
        h.discard(9999);
        std::printf(" %u\n", static_cast<unsigned>(h()));
    }
    return 0;
}
""".replace("%PREFIX%", str(PREFIX))


def main() -> None:
    seeds = [5489] + [m * 131 + n * 17 + d for m, n, d in SHAPES]
    with tempfile.TemporaryDirectory() as tmp:
        src = Path(tmp) / "mt.cpp"
        exe = Path(tmp) / "mt"
        src.write_text(PROGRAM)
        subprocess.run(["g++", "-O2", "-std=c++17", str(src), "-o", str(exe)], check=True)
        out = subprocess.run([str(exe)] + [str(s) for s in seeds], check=True, capture_output=True,
                             text=True).stdout
    entries = []
    for line in out.strip().splitlines():
        values = [int(x) for x in line.split()]
        entries.append({"seed": values[0], "first": values[1:1 + PREFIX], "output_10000": values[-1]})
    version = subprocess.run(["g++", "--version"], check=True, capture_output=True, text=True).stdout.splitlines()[0]
    fixture = {"generator": "std::mt19937 (libstdc++)", "compiler": version, "shapes": SHAPES,
               "entries": entries}
    (HERE / "mt19937_libstdcxx.json").write_text(json.dumps(fixture, separators=(",", ":")) + "\n")
    print(f"wrote {len(entries)} seeds to {HERE / 'mt19937_libstdcxx.json'}")


if __name__ == "__main__":
    main()
