"""kadconv's typed custom operators (torch.library): the fake implementations
give the right output shapes and memory formats under FakeTensorMode (no GPU
needed), as torch.compile / export need to trace through the fast path."""
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import kadconv  # noqa: F401  (registers the operators)
from kadconv import library


class _Shape:
    def __init__(self, cout, stride=1):
        self.cout, self.stride = cout, stride

    def out_shape(self, h, w):
        return self.cout, (h - 1) // self.stride + 1, (w - 1) // self.stride + 1


def test_layer_fwd_fake_shapes():
    h1 = library.register_plan(_Shape(24))
    h2 = library.register_plan(_Shape(8, stride=2))
    try:
        with FakeTensorMode():
            x = torch.empty(2, 16, 9, 13)
            y = torch.ops.kadconv.layer_fwd(x, h1)
            assert tuple(y.shape) == (2, 24, 9, 13) and y.is_contiguous()
            xc = torch.empty(2, 16, 9, 13).contiguous(memory_format=torch.channels_last)
            z = torch.ops.kadconv.layer_fwd(xc, h2)
            assert tuple(z.shape) == (2, 8, 5, 7) and z.is_contiguous(memory_format=torch.channels_last)
    finally:
        library.release_plan(h1)
        library.release_plan(h2)


def test_deform_conv2d_fake_shapes():
    with FakeTensorMode():
        x = torch.empty(2, 5, 11, 13)
        w = torch.empty(7, 5, 3, 3)
        off = torch.empty(2, 18, 6, 7)
        y = torch.ops.kadconv.deform_conv2d(x, off, w, None, 2, 2, 1, 1, 1, 1, None)
        assert tuple(y.shape) == (2, 7, 6, 7)


def test_deform_conv2d_op_cpu_matches_functional():
    """The registered operator's eager path equals kadconv.deform_conv2d (CPU restatement here)."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 4, 6, 7, generator=g, dtype=torch.float64)
    off = torch.randn(1, 18, 6, 7, generator=g, dtype=torch.float64)
    w = torch.randn(3, 4, 3, 3, generator=g, dtype=torch.float64)
    m = torch.rand(1, 9, 6, 7, generator=g, dtype=torch.float64)
    a = torch.ops.kadconv.deform_conv2d(x, off, w, None, 1, 1, 1, 1, 1, 1, m)
    b = kadconv.deform_conv2d(x, off, w, None, padding=1, mask=m)
    assert torch.equal(a, b)
