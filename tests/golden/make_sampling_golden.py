"""Golden draws of the reference's random stream, written from the C++ standard
library itself: std::mt19937(seed) and std::uniform_real_distribution<float>(0, 1)
(what llama_generate_cpu_impl uses, src/models/llama_model.cpp:1556 and :1494),
compiled here with g++ against libstdc++.  Run from the repo root:

    python tests/golden/make_sampling_golden.py

Writes tests/golden/sampling_uniforms.json: per seed, the first 256 raw 32-bit
outputs and the first 256 float draws (as their IEEE bit patterns)."""
import json
import subprocess
import sys
import tempfile
from pathlib import Path

SEEDS = [42, 5489, 1, 123456789]
N = 256
SRC = r"""
#include <cstdio>
#include <cstring>
#include <cstdint>
#include <random>
int main(int argc, char** argv) {
    const unsigned seed = (unsigned)strtoul(argv[1], nullptr, 10);
    const int n = atoi(argv[2]);
    std::mt19937 raw(seed);
    for (int i = 0; i < n; i++) printf("%u%c", (unsigned)raw(), i + 1 < n ? ' ' : '\n');
    std::mt19937 g(seed);
    std::uniform_real_distribution<float> d(0.f, 1.f);
    for (int i = 0; i < n; i++) {
        float x = d(g);
        uint32_t b;
        memcpy(&b, &x, 4);
        printf("%u%c", b, i + 1 < n ? ' ' : '\n');
    }
}
"""


def main() -> int:
    out = Path(__file__).resolve().parent / "sampling_uniforms.json"
    with tempfile.TemporaryDirectory() as d:
        src, exe = Path(d) / "g.cpp", Path(d) / "g"
        src.write_text(SRC)
        subprocess.run(["g++", "-O2", "-std=c++17", str(src), "-o", str(exe)], check=True)
        ver = subprocess.run(["g++", "--version"], capture_output=True, text=True).stdout.splitlines()[0]
        data = {"compiler": ver, "n": N, "seeds": {}}
        for s in SEEDS:
            lines = subprocess.run([str(exe), str(s), str(N)], capture_output=True, text=True,
                                   check=True).stdout.splitlines()
            data["seeds"][str(s)] = {"mt19937": [int(v) for v in lines[0].split()],
                                     "uniform_f32_bits": [int(v) for v in lines[1].split()]}
    out.write_text(json.dumps(data))
    print(f"wrote {out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
