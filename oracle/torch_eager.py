"""PyTorch CPU eager forms of the five hot-path ops - TEST INFRASTRUCTURE ONLY.

The reference checks every kernel against torch eager on the same inputs
(tests/test_vector_add.py:30, tests/test_softmax_layernorm.py:47-62,
tests/test_matmul.py:52-71, examples/05_fused_attention.py:67-73). These are
those same calls, on the CPU, in fp32 upcasts. bench.py times them on the GPU
host as the reported CPU baseline (never as the thing measured on the GPU);
tests may use them as a second checker beside oracle/newt_oracle.py. No
product code imports this module.
"""

import torch


def vector_add(x, y):
    return x + y


def softmax(x):
    return torch.softmax(x.float(), dim=-1)


def layernorm(x, w, b, eps=1e-5):
    """(y, mean, rstd) from torch.native_layer_norm on fp32 upcasts."""
    n = x.shape[-1]
    y, mean, rstd = torch.native_layer_norm(x.float(), (n,), w.float(), b.float(), eps)
    return y.to(x.dtype), mean.reshape(-1), rstd.reshape(-1)


def matmul(a, b):
    return a.float() @ b.float()


def attention(q, k, v, causal=False, scale=None):
    return torch.nn.functional.scaled_dot_product_attention(
        q.float(), k.float(), v.float(), is_causal=causal, scale=scale)
