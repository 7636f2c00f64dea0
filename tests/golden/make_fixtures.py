"""Writes the small committed fixtures under tests/golden/.

sgemm_srand42_head.json: the first 16 (A, B) pairs of the SGEMM input generator
(srand(42); A[i], B[i] = (rand()%2000 - 1000)/1000.0f interleaved, gpu_workload.c:81-82),
produced through libswitchgpu.so's sgpu_gen_sgemm_inputs on this image's glibc.  The
reference holds no stored vectors for this path; the fixture pins the generator against
drift (a different libc rand(), a changed interleave) between machines.

Run: python tests/golden/make_fixtures.py  (after building the package)
"""
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(HERE)), "switch-l4t-gpu_amd"))

import sgpu  # noqa: E402


def main():
    A, B = sgpu.gen_sgemm_inputs(16, 42)
    with open(os.path.join(HERE, "sgemm_srand42_head.json"), "w") as f:
        json.dump({"seed": 42, "A": [float(v) for v in A], "B": [float(v) for v in B]}, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
