"""The engine's registered torch operators (w8a8.torch_ops) without a GPU: every operator exists
under torch.ops.w8a8 with the schema its wrappers call, and its fake implementation gives the
output shape and dtype the kernel writes (checked on meta tensors, which is what torch.compile's
tracing sees)."""
import re

import torch

from w8a8 import torch_ops  # noqa: F401  (registers the operators)


def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(shape, dtype=dtype, device="meta")


def test_operators_are_registered_with_their_schemas():
    names = ("mm_i8", "linear", "gemv", "rms_norm", "attention", "attention_decode")
    for n in names:
        assert hasattr(torch.ops.w8a8, n), n
    schema = str(torch.ops.w8a8.mm_i8.default._schema)
    assert re.search(r"Tensor\(a\d*!\) c\)", schema) and schema.endswith("-> ()"), schema  # c is written in place
    for n in names[1:]:
        assert "!)" not in str(getattr(torch.ops.w8a8, n).default._schema), n  # no input is written


def test_fake_shapes():
    w = meta(1000, dtype=torch.int8)
    sw = meta(12288, dtype=torch.float32)
    y = torch.ops.w8a8.linear(meta(512, 1536), w, sw, 12288, 1536, 6144, "gelu", None, None, 1e-6)
    assert y.shape == (512, 6144) and y.dtype == torch.bfloat16
    y = torch.ops.w8a8.linear(meta(77, 6144), w, meta(1536, dtype=torch.float32), 1536, 6144, 0, "residual",
                              meta(77, 1536), None, 1e-6)
    assert y.shape == (77, 1536)
    y = torch.ops.w8a8.gemv(meta(4, 1536), w, 262144, 1536, meta(262144))
    assert y.shape == (4, 262144) and y.dtype == torch.bfloat16
    y = torch.ops.w8a8.rms_norm(meta(40, 256), meta(256), 1e-6)
    assert y.shape == (40, 256)
    y = torch.ops.w8a8.attention(meta(8, 3658, 512), meta(1, 3658, 512), meta(1, 3658, 512), 0, 0, 1.0)
    assert y.shape == (8, 3658, 512)
    y = torch.ops.w8a8.attention_decode(meta(8, 256), meta(1, 100, 256), meta(1, 100, 256), 99, 512, 1.0)
    assert y.shape == (8, 256)
    c = meta(512, 2560, dtype=torch.int32)
    assert torch.ops.w8a8.mm_i8(meta(512, 1536, dtype=torch.int8), w, 2560, 1536, c) is None


def test_helpers_call_the_eager_path_outside_tracing():
    assert not torch_ops.tracing()
