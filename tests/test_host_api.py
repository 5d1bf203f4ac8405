"""Host-side behaviour of the kadconv package (no GPU needed): the reference's
API surface (KAD-Conv/kadconv/__init__.py:1-4, fast.py:68-118) and its error
behaviour."""
import pytest
import torch
import torch.nn as nn

import kadconv
from kadconv import fast
from kadconv import synthetic as S
from oracle import kadconv_oracle as O


def test_public_api_names():
    for name in ['KADConv', 'DSC', 'LCSA', 'enable_fast_inference', 'disable_fast_inference']:
        assert hasattr(kadconv, name)


def test_state_dict_keys_match_oracle_layout():
    m = kadconv.KADConv(256, se_min_hidden=64)
    sd = S.make_kadconv_state(256, se_min_hidden=64)
    ours = {k for k in m.state_dict() if not k.endswith('num_batches_tracked')}
    assert ours == set(sd)
    for k, v in sd.items():
        assert m.state_dict()[k].shape == v.shape, k
    assert m.load_state_dict(sd, strict=False).unexpected_keys == []


def test_dsc_init_and_attributes():
    d = kadconv.DSC(10, 12)
    assert d.mask is True and d.stride == (1, 1) and d.padding == 1 and d.kernel_size == 3
    assert torch.count_nonzero(d.conv_offset.weight) == 0 and torch.count_nonzero(d.conv_offset.bias) == 0
    bound = 1 / (10 * 9) ** 0.5
    assert d.weight.abs().max() <= bound


def test_enable_raises_in_training_mode():
    m = kadconv.KADConv(16)
    with pytest.raises(ValueError, match='eval'):
        kadconv.enable_fast_inference(m)


def test_enable_raises_on_cpu_model():
    m = kadconv.KADConv(16).eval()
    with pytest.raises(ValueError, match='GPU'):
        kadconv.enable_fast_inference(m)


def test_layer_discovery_by_class_name():
    class KADC4(nn.Module):  # KAD-CNet's class name for the same layer
        pass

    class DCN_RCA(nn.Module):
        pass

    net = nn.Sequential(nn.Conv2d(3, 3, 1), KADC4(), kadconv.KADConv(8), kadconv.DSC(4, 4))
    names = [type(m).__name__ for m in net.modules() if type(m).__name__ in fast._LAYER_TYPES]
    assert names == ['KADC4', 'KADConv']
    dscs = [type(m).__name__ for m in net.modules() if type(m).__name__ in fast._DSC_TYPES]
    assert dscs == ['DSC'] * 4  # three inside KADConv(8), one standalone
    assert 'DCN_RCA' in fast._DSC_TYPES and 'KADC4_m' in fast._LAYER_TYPES


def test_disable_removes_instance_forward():
    m = kadconv.KADConv(8).eval()
    m.forward = lambda x: x  # what enable_fast_inference installs, in shape
    kadconv.disable_fast_inference(m)
    assert 'forward' not in vars(m)


def test_cpu_deform_rejects_bad_shapes():
    """The CPU deformable conv checks offset and mask shapes as torchvision does."""
    x = torch.randn(1, 4, 5, 5)
    with pytest.raises(ValueError, match='offset shape'):
        kadconv.deform_conv2d(x, torch.zeros(1, 9, 5, 5), torch.zeros(4, 4, 3, 3), padding=1)
    with pytest.raises(ValueError, match='mask shape'):
        kadconv.deform_conv2d(x, torch.zeros(1, 18, 5, 5), torch.zeros(4, 4, 3, 3), padding=1,
                              mask=torch.zeros(1, 8, 5, 5))


def test_kaddown_plain_matches_oracle_on_cpu():
    m = kadconv.KADDown(6, 10)
    sd = S.make_kaddown_state(6, 10, seed=3)
    m.load_state_dict(sd)
    x = torch.randn(2, 6, 24, 16)
    with torch.no_grad():
        got = m(x)
    ref = O.kaddown_forward(sd, x)
    assert torch.allclose(got, ref, atol=1e-6, rtol=1e-5)


def test_se_and_conv_blocks_plain_on_cpu():
    se = kadconv.SqueezeExcitation(32, reduction=16)
    x = torch.randn(2, 32, 5, 6)
    p = se.state_dict()
    ref = O.se_forward(x, p['fc.0.weight'], p['fc.0.bias'], p['fc.2.weight'], p['fc.2.bias'])
    assert torch.allclose(se(x), ref, atol=1e-6)
    conv = nn.Conv2d(8, 6, 1, bias=False)
    bn = nn.BatchNorm2d(6).eval()
    with torch.no_grad():
        bn.running_mean.uniform_(-1, 1)
        bn.running_var.uniform_(0.5, 2)
    blk = kadconv.Conv1x1SiLU.from_conv_bn(conv, bn)
    x = torch.randn(1, 8, 4, 4)
    assert torch.allclose(blk(x), torch.nn.functional.silu(bn(conv(x))), atol=1e-5)


def test_missing_library_raises(monkeypatch, tmp_path):
    from kadconv import _ext
    monkeypatch.setattr(_ext, '_LIB_PATH', str(tmp_path / 'nope.so'))
    monkeypatch.setattr(_ext, '_lib', None)
    with pytest.raises(_ext.KadExtensionError):
        _ext.load()
