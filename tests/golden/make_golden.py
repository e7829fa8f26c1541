"""Writes the committed fixtures of tests/golden/ (run in the build container,
where the reference tree is present):

  q8_0_ggml.npz   inputs and the outputs of ggml's own quantize_row_q8_0 (x86
                  AVX2 path), quantize_row_q8_0_ref and dequantize_row_q8_0,
                  compiled from the reference sources in place (oracle/_ref)
  attn_small.npz  a small paged-attention case and its float64 brute-force
                  output (softmax(scale*qK^T + mask) V from the definition)

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

from oracle import oracle  # noqa: E402
from helpers import brute_force, make_case  # noqa: E402


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref could not be built: the reference tree is required")
    rng = np.random.default_rng(20261201)
    x = rng.standard_normal((48, 128)).astype(np.float32)
    x[0, :32] = 0.0
    x[1, :32] = 0.0
    x[1, 0] = 127.0
    x[1, 1:8] = [2.5, -2.5, 0.5, 1.5, -0.5, 126.5, 3.5]
    x[2] *= 1e-30
    x[3] *= 3e4
    q_x86 = np.zeros((48, 128 // 32 * 34), np.uint8)
    q_ref = np.zeros_like(q_x86)
    deq = np.zeros_like(x)
    ref.ref_quantize_row_q8_0_x86(x.ctypes.data, q_x86.ctypes.data, x.size)
    ref.ref_quantize_row_q8_0_scalar(x.ctypes.data, q_ref.ctypes.data, x.size)
    ref.ref_dequantize_row_q8_0(q_x86.ctypes.data, deq.ctypes.data, x.size)
    np.savez_compressed(HERE / "q8_0_ggml.npz", x=x, q_x86=q_x86, q_ref=q_ref, deq_x86=deq)

    c = make_case(np.random.default_rng(7), 8, 2, 64, [40, 70, 16], [1, 3, 2], num_blocks=16)
    out = brute_force(c)
    np.savez_compressed(HERE / "attn_small.npz", q=c.q, k_pool=c.k_pool, v_pool=c.v_pool, bt=c.bt,
                        seq_lens=c.seq_lens, seq_idx=c.seq_idx, pos=c.pos, Hkv=c.Hkv, scale=c.scale,
                        n_swa=c.n_swa, out_f64=out)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
