"""Writes tests/golden/w8a8_golden.npz -- small input/output vectors for the W8A8
path, produced by the CPU oracle (oracle/, a restatement of aikit's Go linalg).

The reference holds no W8A8 fixture of its own (its testdata/*.json are HF f32
goldens for absent checkpoints), so these vectors are self-generated. They are
not trusted on the oracle's word: tests/test_oracle.py checks each one against
what the mathematics fixes independently of the oracle (numpy int64 dots, the
reference's own test vectors from encoder/quant_test.go:187-201 and
gpu/cuda_vit_test.go:154-310, the half-away-from-zero tie rule, long-double erf).

Run:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402

OUT = os.path.join(HERE, "w8a8_golden.npz")


def quant_rows():
    """Ragged quantization cases: (name, row)."""
    g = np.random.Generator(np.random.PCG64(3))
    cases = [
        ("ref_extreme", np.array([1.0, -1.0, 0.0, 0.0], np.float32)),  # encoder/quant_test.go:187-201
        ("zero", np.zeros(8, np.float32)),  # encoder/quant_test.go:165-185; gpu/cuda_vit_test.go:159-161
        ("neg_zero", np.array([-0.0, 0.0, -0.0], np.float32)),
        ("ties", np.array([127, 0.5, 1.5, 2.5, -0.5, -2.5, 126.5, -126.5], np.float32)),
        ("nan_ignored", np.array([np.nan, 1.0, -2.0, 0.25], np.float32)),
        ("inf_row", np.array([np.inf, 1.0, -3.0], np.float32)),
        ("subnormal", np.array([1e-40, -1e-40, 5e-41, 0.0], np.float32)),
        ("single", np.array([-3.25], np.float32)),
    ]
    # gpu/cuda_vit_test.go:157-162: 12 rows x 97, N(0,1)*2, row 5 all zero.
    x = (g.standard_normal((12, 97)) * 2).astype(np.float32)
    x[5] = 0
    for r in range(12):
        cases.append((f"vit_row{r}", x[r].copy()))
    return cases


def main():
    data = {}
    rows = quant_rows()
    flat = np.concatenate([r for _, r in rows]).astype(np.float32)
    offs = np.cumsum([0] + [len(r) for _, r in rows]).astype(np.int64)
    codes_act, scales_act, codes_w, scales_w = [], [], [], []
    for _, r in rows:
        q, s = oracle.quantize_row(r, 0.0)
        codes_act.append(q)
        scales_act.append(s)
        q, s = oracle.quantize_row(r, 1.0)
        codes_w.append(q)
        scales_w.append(s)
    data.update(
        quant_names=np.array([n for n, _ in rows]),
        quant_rows=flat,
        quant_offsets=offs,
        quant_codes_act=np.concatenate(codes_act),
        quant_scales_act=np.array(scales_act, np.float32),
        quant_codes_w=np.concatenate(codes_w),
        quant_scales_w=np.array(scales_w, np.float32),
    )

    # Integer GEMM + rescale at the reference's own shapes (gpu/cuda_vit_test.go:233):
    # (M, N, K) = (1,8,16), (16,32,32), (17,33,65); int8 in [-127,127], scales N(0,1)*0.01.
    g = np.random.Generator(np.random.PCG64(4))
    for i, (M, N, K) in enumerate([(1, 8, 16), (16, 32, 32), (17, 33, 65)]):
        A = g.integers(-127, 128, size=(M, K), dtype=np.int8)
        B = g.integers(-127, 128, size=(N, K), dtype=np.int8)
        a_s = (g.standard_normal(M) * 0.01).astype(np.float32)
        b_s = (g.standard_normal(N) * 0.01).astype(np.float32)
        data[f"gemm{i}_A"], data[f"gemm{i}_B"] = A, B
        data[f"gemm{i}_as"], data[f"gemm{i}_bs"] = a_s, b_s
        data[f"gemm{i}_acc"] = oracle.acc_i32(A, B, M, K, N)
        data[f"gemm{i}_dst"] = oracle.w8a8_span(A, a_s, B, b_s, M, K, N)

    # Full linears (quantize -> GEMM -> bias -> GELU) on f32 activations.
    g = np.random.Generator(np.random.PCG64(5))
    for i, (M, K, N, act, with_bias) in enumerate([(5, 70, 40, 1, True), (3, 64, 33, 0, False),
                                                   (9, 130, 65, 1, True)]):
        a = (g.standard_normal((M, K)) * 1.5).astype(np.float32)
        a[min(2, M - 1)] = 0  # an all-zero activation row: scale 0, output = bias
        w = (g.standard_normal((N, K)) * 0.05).astype(np.float32)
        wq, ws = oracle.quantize_rows_weights(w, N, K)
        b = (g.standard_normal(N) * 0.1).astype(np.float32) if with_bias else None
        data[f"lin{i}_a"], data[f"lin{i}_wq"], data[f"lin{i}_ws"] = a, wq, ws
        data[f"lin{i}_bias"] = b if b is not None else np.zeros(0, np.float32)
        data[f"lin{i}_act"] = np.array(act, np.int32)
        data[f"lin{i}_dst"] = oracle.w8a8_linear(a, wq, ws, b, act, M, K, N)

    # GELU at hand-picked points, including every branch of ErfF32.
    gx = np.array([0.0, -0.0, 1e-30, 0.5, -0.5, 1.0, 1.4142135, 1.4142137, -1.7, 3.0, -3.0, 5.656854,
                   5.656855, -5.656855, 10.0, -10.0, 100.0, -100.0, 2.5e-3, -7.0e-2], np.float32)
    data["gelu_x"], data["gelu_y"] = gx, oracle.gelu(gx)
    np.savez_compressed(OUT, **data)
    print("wrote", OUT, sum(v.nbytes for v in data.values()), "bytes")


if __name__ == "__main__":
    main()
