"""Write the golden fixtures for the hot-path parity tests.

The reference's oracle is PyTorch eager on seeded inputs (its tests compare
every kernel against torch: tests/test_vector_add.py:30,
tests/test_softmax_layernorm.py:47-62, tests/test_matmul.py:52-71,
examples/05_fused_attention.py:67-73). This script evaluates those same torch
ops on the CPU, in float64 where the reference upcasts, on small seeded inputs
shaped like the reference's own test cases, and stores inputs and outputs as
.npz files next to it. Run: python tests/golden/make_golden.py
"""

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def gen(shape, seed, scale=1.0, mean=0.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale + mean).to(dtype)


def save(name, **arrays):
    path = os.path.join(HERE, f"{name}.npz")
    np.savez_compressed(path, **{k: (v.float().numpy() if torch.is_tensor(v) else v)
                                 for k, v in arrays.items()})
    print("wrote", path)


def main():
    # vector add: n=12345 exercises the masked tail (tests/test_vector_add.py:23)
    x, y = gen(12345, 0), gen(12345, 1)
    save("vector_add_12345", x=x, y=y, out=x + y)

    # softmax: the reference test shapes incl. non-pow2 columns (test_softmax_layernorm.py:41)
    for M, N in [(8, 128), (32, 781)]:
        x = gen((M, N), 0, scale=4.0)
        save(f"softmax_{M}x{N}", x=x, out=torch.softmax(x.double(), dim=-1))

    # layernorm: fp16 input like config 3, saved mean / rstd (native_layer_norm)
    for M, N in [(16, 300), (8, 128)]:
        x = gen((M, N), 0, dtype=torch.float16)
        w = gen(N, 2, scale=0.1, mean=1.0, dtype=torch.float16)
        b = gen(N, 3, scale=0.1, dtype=torch.float16)
        y, mean, rstd = torch.native_layer_norm(x.double(), (N,), w.double(), b.double(), 1e-5)
        save(f"layernorm_{M}x{N}", x=x, w=w, b=b, out=y, mean=mean.reshape(-1),
             rstd=rstd.reshape(-1))

    # matmul: tests/test_matmul.py shapes (incl. ragged 300x200x100)
    for M, N, K in [(64, 64, 32), (300, 200, 100)]:
        a = gen((M, K), 4, scale=K ** -0.5, dtype=torch.float16)
        b = gen((K, N), 5, scale=K ** -0.5, dtype=torch.float16)
        save(f"matmul_{M}x{N}x{K}", a=a, b=b, out=a.double() @ b.double())

    # attention: tiny [1, 2, 64, 32] heads, causal and not (examples/05)
    q, k, v = (gen((1, 2, 64, 32), s, dtype=torch.bfloat16) for s in (6, 7, 8))
    for causal in (False, True):
        o = torch.nn.functional.scaled_dot_product_attention(
            q.double(), k.double(), v.double(), is_causal=causal, scale=32 ** -0.5)
        save(f"attention_1x2x64x32_{'causal' if causal else 'full'}", q=q, k=k, v=v, out=o)


if __name__ == "__main__":
    main()
