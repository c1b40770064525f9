"""Writes the small golden fixtures in this folder from the CPU oracle.

Each .npz holds seeded inputs (xorshift generator of src/lora.rs:80-92, per-
tensor sub-seeds) and the float64 oracle output `y`. Regenerate with
`python tests/golden/make_golden.py`; test_oracle.py checks they still
reproduce, and the GPU tests check the HIP kernels against them.
cfg1 (K = N = 2048) is too large to commit; cfg1_sha256.json records the
SHA-256 of its generated inputs and f64 output instead.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle as O  # noqa: E402

E = np.zeros(0, np.uint32)


def gptq(name, seed, K, N, gs, zeros=False, act=False, M=0, kind="matvec"):
    c = O.gptq_case(seed, K, N, gs, zeros=zeros, act_order=act, M=M)
    extra = {}
    x = c["x"]
    if kind == "silu":
        a = O.normal_f32(seed * 16 + 7, K if M == 0 else M * K).reshape(x.shape)
        b = O.normal_f32(seed * 16 + 8, K if M == 0 else M * K).reshape(x.shape)
        extra = {"a": a, "b": b}
        x = O.silu_mul_f64(a, b)
    y = O.gptq_matvec_f64(x, c["qweight"], c["scales"], K, N, gs, qzeros=c["qzeros"], g_idx=c["g_idx"])
    np.savez_compressed(os.path.join(HERE, name), kind=kind, K=K, N=N, gs=gs, x=c["x"], qweight=c["qweight"],
                        scales=c["scales"], qzeros=c["qzeros"] if zeros else E,
                        g_idx=c["g_idx"] if act else E.astype(np.int32), y=y, **extra)


def int8(name, seed, K, N, M):
    c = O.int8_case(seed, K, N, M=M)
    y = O.int8_matvec_f64(c["x"], c["w"], c["scale"], K, N)
    np.savez_compressed(os.path.join(HERE, name), kind="int8", K=K, N=N, x=c["x"], w=c["w"], scale=c["scale"], y=y)


def main():
    gptq("i4_k256_n64_sym.npz", 21, 256, 64, 128)
    gptq("i4_k256_n64_zeros.npz", 22, 256, 64, 128, zeros=True)
    gptq("i4_k256_n64_actorder.npz", 23, 256, 64, 128, act=True)
    gptq("i4_k256_n64_zeros_actorder.npz", 24, 256, 64, 128, zeros=True, act=True)
    gptq("i4_k256_n64_g64_m4.npz", 25, 256, 64, 64, M=4)
    gptq("i4_k256_n64_silu.npz", 26, 256, 64, 128, kind="silu")
    int8("i8_k256_n64_m8.npz", 27, 256, 64, 8)
    c = O.gptq_case(0, 2048, 2048, 128)
    y = O.gptq_matvec_f64(c["x"], c["qweight"], c["scales"], 2048, 2048, 128)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()  # noqa: E731
    with open(os.path.join(HERE, "cfg1_sha256.json"), "w") as f:
        json.dump({"seed": 0, "K": 2048, "N": 2048, "gs": 128, "x": h(c["x"]), "qweight": h(c["qweight"]),
                   "scales": h(c["scales"]), "y_f64": h(y)}, f, indent=1)


if __name__ == "__main__":
    main()
