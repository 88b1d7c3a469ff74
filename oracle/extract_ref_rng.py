"""Test infrastructure (the oracle's pins): prints, as HIP source, the reference's four Drop
generators -- the rng_init / rng_u32 pairs and rng_uniform of the NVRTC prelude text in
src/tkm_gpu.cu:751-794, as they stand there -- for oracle/ref_rng_harness.hip.

Usage: python3 extract_ref_rng.py /root/reference > oracle/_ref/ref_rng.inc
The prelude is a sequence of C string literals, one per source line; the lines from
`struct RngXorshift32` up to the one before `rng_normal2` are read and unescaped.  The
output goes only under oracle/_ref/ (not in the repository); it compiles as HIP device code
without any stand-in, since HIP provides the intrinsics it uses (__umulhi).
"""
import ast
import sys


def main(ref: str) -> None:
    lines = open(f"{ref}/src/tkm_gpu.cu").read().splitlines()
    start = next(i for i, ln in enumerate(lines) if ln.lstrip().startswith('"struct RngXorshift32'))
    end = next(i for i in range(start, len(lines)) if "rng_normal2" in lines[i])
    text = "".join(ast.literal_eval(ln.strip()) for ln in lines[start:end])
    for name in ("RngXorshift32", "RngWangXorshift32", "RngPcg32", "RngPhilox", "rng_uniform"):
        assert name in text, name
    sys.stdout.write(f"/* src/tkm_gpu.cu lines {start + 1}-{end} (prelude text), extracted by extract_ref_rng.py */\n")
    sys.stdout.write(text)


if __name__ == "__main__":
    main(sys.argv[1])
