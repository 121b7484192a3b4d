"""Writes the golden fixtures of tests/golden/ from the reference's own CPU
functions (oracle/_ref/libgqref.so, compiled from the reference sources where
they lie; see oracle/Makefile).  Run in the build container, where the reference
tree exists:  python tests/golden/make_golden.py

Fixtures (inputs and expected outputs only, .npz):
  q4k_ref.npz   96 random Q4_K blocks (with fp16 edge values in d/dmin) and the
                reference dequantize_q4_k_block output (weight_loader.cpp:125-156)
  q6k_ref.npz   48 random Q6_K blocks and dequantize_q6_k_block output (:158-177)
  fp16_ref.npz  fp16_to_fp32 (weight_loader.cpp:91-110) of all 65536 inputs
  gemm_ref.npz  CpuReference::gemm (cpu_reference.hpp:56-66) on a 5x7x9 case
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402

SPECIAL16 = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0x7C00, 0xFC00, 0x7E00, 0x3C00, 0x8001, 0x1234]


def main():
    R = O.ref()
    if R is None:
        raise SystemExit("oracle/_ref/libgqref.so not built (needs the reference tree)")
    rng = np.random.default_rng(20240601)

    blocks = rng.integers(0, 256, size=(96, 144), dtype=np.uint8)
    for i, h in enumerate(SPECIAL16):
        blocks[i, 0:2] = np.frombuffer(np.uint16(h).tobytes(), np.uint8)
        blocks[i, 2:4] = np.frombuffer(np.uint16(SPECIAL16[-1 - i]).tobytes(), np.uint8)
    blocks[12:, 0:2] = (np.abs(rng.standard_normal(84)) * 0.01).astype(np.float16).view(np.uint8).reshape(84, 2)
    blocks[12:, 2:4] = (np.abs(rng.standard_normal(84)) * 0.01).astype(np.float16).view(np.uint8).reshape(84, 2)
    out = np.empty(96 * 256, np.float32)
    R.gqref_dequant_q4_k(blocks.ctypes.data, 96, out.ctypes.data)
    np.savez_compressed(os.path.join(HERE, "q4k_ref.npz"), blocks=blocks, out=out)

    b6 = rng.integers(0, 256, size=(48, 210), dtype=np.uint8)
    b6[:, 208:210] = (np.abs(rng.standard_normal(48)) * 0.01).astype(np.float16).view(np.uint8).reshape(48, 2)
    out6 = np.empty(48 * 256, np.float32)
    R.gqref_dequant_q6_k(b6.ctypes.data, 48, out6.ctypes.data)
    np.savez_compressed(os.path.join(HERE, "q6k_ref.npz"), blocks=b6, out=out6)

    h = np.arange(65536, dtype=np.uint32)
    f = np.array([R.gqref_fp16_to_fp32(int(i)) for i in h], dtype=np.float32)
    np.savez_compressed(os.path.join(HERE, "fp16_ref.npz"), out=f)

    A = rng.standard_normal((5, 9)).astype(np.float32)
    B = rng.standard_normal((9, 7)).astype(np.float32)
    C = np.empty((5, 7), np.float32)
    R.gqref_gemm(A.ctypes.data, B.ctypes.data, C.ctypes.data, 5, 7, 9)
    np.savez_compressed(os.path.join(HERE, "gemm_ref.npz"), A=A, B=B, C=C)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
