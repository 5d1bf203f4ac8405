"""KAD-CNet-S on the CPU: the model dictionary against the reference's YAML,
the channel plan, the plain forward against the oracle, Conv-BN fusion, and
pins of the oracle's DDetect decode and NMS (closed forms and hand-made
known answers)."""
import os

import numpy as np
import pytest
import torch

import kadcnet
from oracle import kadcnet_oracle as KO

REF_CFG = '/root/reference/KAD-CNet/configs'


@pytest.mark.parametrize('name,cfg', [('dior_s_base.yaml', kadcnet.DIOR_S_BASE), ('dior_s_mgl.yaml', kadcnet.DIOR_S_MGL)])
def test_model_dictionary_matches_reference_yaml(name, cfg):
    """DIOR_S_BASE / DIOR_S_MGL row for row against KAD-CNet/configs/*.yaml (read as
    text with yaml.safe_load where the reference tree is present)."""
    path = os.path.join(REF_CFG, name)
    if not os.path.exists(path):
        pytest.skip('reference tree not present')
    import yaml
    ref = yaml.safe_load(open(path))
    for k in ('nc', 'depth_multiple', 'width_multiple', 'anchors', 'ch'):
        assert cfg[k] == ref[k], k
    assert cfg['backbone'] == ref['backbone']
    assert cfg['head'] == ref['head']
    assert cfg.get('mgl_encoder_channels') == ref.get('mgl_encoder_channels')


@pytest.fixture(scope='module')
def model():
    return kadcnet.build_kadcnet_s(seed=0)


def test_channel_plan(model):
    """Width 1.1 with make_divisible(., 8) ceiling (utils/general.py:660-664): the
    backbone 40/72/72/144/144/216/216/288/288, 42 KADC4 layers (6 per GELAN block,
    126 DSCs) of widths 32 / 48 / 64, DDetect inputs 144/216/288."""
    plan = KO.channel_plan(kadcnet.DIOR_S_BASE)
    assert plan[:10] == [40, 72, 72, 144, 144, 216, 216, 288, 288, 288]
    x = torch.zeros(1, 3, 256, 256)
    outs = []
    with torch.no_grad():
        cur = x
        for m in model.model[:-1]:
            if m.f != -1:
                cur = outs[m.f] if isinstance(m.f, int) else [cur if j == -1 else outs[j] for j in m.f]
            cur = m(cur)
            outs.append(cur)
    assert [o.shape[1] for o in outs] == plan[:-1]
    det = model.model[-1]
    assert [m[0].conv.in_channels for m in det.cv2] == [144, 216, 288]
    kadc = [m for m in model.modules() if type(m).__name__ == 'KADC4']
    assert len(kadc) == 42
    assert sum(1 for m in model.modules() if type(m).__name__ == 'DSC') == 126
    assert sorted({m.convs[0][0].weight.shape[1] for m in kadc}) == [32, 48, 64]
    assert [float(s) for s in model.stride] == [8.0, 16.0, 32.0]


def test_state_dict_names_follow_reference(model):
    keys = set(model.state_dict())
    for k in ('model.0.conv.weight', 'model.0.bn.running_var', 'model.3.cv1.conv.weight',
              'model.4.cv2.0.m.0.convs.0.1.RCA_mask.excite.4.weight', 'model.4.cv2.0.cv3.bn.weight',
              'model.9.cv5.conv.weight', 'model.22.cv2.0.2.weight', 'model.22.cv3.2.2.bias', 'model.22.dfl.conv.weight',
              'model.21.cv3.0.m.2.fc.2.2.bias', 'model.21.cv3.0.m.2.weight.1.0.weight'):
        assert k in keys, k


def test_plain_forward_matches_oracle(model):
    m = kadcnet.build_kadcnet_s(seed=0).double()
    x = torch.rand(1, 3, 128, 160, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    with torch.no_grad():
        y, heads = m(x)
    sd = dict(m.state_dict())
    yo, ho = KO.kadcnet_forward(sd, kadcnet.DIOR_S_BASE, x)
    assert torch.allclose(y, yo, rtol=0, atol=1e-9 * yo.abs().max().item())
    for a, b in zip(heads, ho):
        assert torch.allclose(a, b, rtol=0, atol=1e-9 * b.abs().max().item())


def test_fuse_equals_unfused():
    a = kadcnet.build_kadcnet_s(seed=3).double()
    b = kadcnet.build_kadcnet_s(seed=3).double().fuse()
    assert not any(hasattr(m, 'bn') for m in b.modules() if type(m).__name__ == 'Conv')
    x = torch.rand(1, 3, 128, 128, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    with torch.no_grad():
        ya, _ = a(x)
        yb, _ = b(x)
    assert torch.allclose(ya, yb, rtol=0, atol=1e-9 * ya.abs().max().item())
    # the oracle reads the fused layout (conv.bias, no bn.*) too
    yo, _ = KO.kadcnet_forward(dict(b.state_dict()), kadcnet.DIOR_S_BASE, x)
    assert torch.allclose(yb, yo, rtol=0, atol=1e-9 * yo.abs().max().item())


def test_oracle_decode_one_hot_bins():
    """With one bin logit far above the rest on each side, the DFL expectation is
    that bin index, so the boxes follow in closed form: anchor (x + 0.5, y + 0.5),
    x1 = ax - l, x2 = ax + r, xywh * stride; classes are sigmoid(logit)."""
    g = torch.Generator().manual_seed(0)
    nc, H, W, s = 3, 2, 3, 8.0
    bins = torch.randint(0, 16, (1, 4, H, W), generator=g)
    head = torch.full((1, 64 + nc, H, W), -60.0, dtype=torch.float64)
    for j in range(4):
        head[:, 16 * j:16 * (j + 1)].scatter_(1, bins[:, j:j + 1], 60.0)
    cls = torch.randn(1, nc, H, W, generator=g, dtype=torch.float64)
    head[:, 64:] = cls
    y = KO.ddetect_decode([head], [s], nc)
    d = bins[0].double().reshape(4, -1)
    gy, gx = torch.meshgrid(torch.arange(H) + 0.5, torch.arange(W) + 0.5, indexing='ij')
    ax, ay = gx.reshape(-1).double(), gy.reshape(-1).double()
    exp_box = torch.stack(((ax - d[0] + ax + d[2]) / 2, (ay - d[1] + ay + d[3]) / 2, d[0] + d[2], d[1] + d[3])) * s
    assert torch.allclose(y[0, :4], exp_box, atol=1e-9)
    assert torch.allclose(y[0, 4:], torch.sigmoid(cls.reshape(nc, -1)), atol=1e-12)


def test_oracle_decode_matches_reference_module_path(model):
    """The oracle decode against the model's own DDetect tail (DFL 1x1 conv of a
    softmax, make_anchors, dist2bbox), on random heads."""
    det = model.model[-1]
    g = torch.Generator().manual_seed(5)
    heads = [torch.randn(2, 84, h, w, generator=g) for h, w in ((8, 10), (4, 5), (2, 3))]
    box, cls = torch.cat([h.view(2, 84, -1) for h in heads], 2).split((64, 20), 1)
    anchors, strides = (t.transpose(0, 1) for t in kadcnet.make_anchors(heads, det.stride, 0.5))
    ref = torch.cat((kadcnet.dist2bbox(det.dfl(box), anchors.unsqueeze(0), xywh=True, dim=1) * strides,
                     cls.sigmoid()), 1)
    got = KO.ddetect_decode([h.double() for h in heads], [8.0, 16.0, 32.0], 20)
    assert torch.allclose(got, ref.double(), atol=1e-4, rtol=1e-5)


def test_oracle_nms_known_answers():
    # 0 and 1 overlap with IoU 81/119 = 0.68; 2 is disjoint; 3 touches 0 with IoU exactly 0.5
    boxes = np.array([[0, 0, 10, 10], [1, 1, 11, 11], [20, 20, 30, 30], [5, 0, 15, 10], [0, 0, 10, 10]], float)
    # box 3 vs box 0: inter 50, union 150 -> 1/3; box 4 duplicates box 0 with a lower score
    scores = np.array([0.9, 0.8, 0.7, 0.6, 0.5])
    assert KO.nms(boxes, scores, 0.5) == [0, 2, 3]
    assert KO.nms(boxes, scores, 0.3) == [0, 2]
    assert KO.nms(boxes, scores, 0.7) == [0, 1, 2, 3]
    # IoU exactly at the threshold is kept ("> thr" suppresses)
    assert KO.nms(np.array([[0, 0, 2, 1], [1, 0, 3, 1]], float), np.array([1.0, 0.5]), 1 / 3) == [0, 1]
    # ties in score keep index order
    assert KO.nms(np.array([[0, 0, 1, 1], [0, 0, 1, 1]], float), np.array([0.5, 0.5]), 0.5) == [0]
    assert KO.nms(np.zeros((0, 4)), np.zeros(0), 0.5) == []


def test_oracle_nms_matches_pairwise_definition():
    """Random overlapping boxes: every dropped box overlaps (IoU > thr) a kept box
    with a higher rank, and no two kept boxes overlap above thr."""
    rng = np.random.default_rng(0)
    n = 300
    xy = rng.uniform(0, 100, (n, 2))
    wh = rng.uniform(5, 30, (n, 2))
    boxes = np.concatenate((xy, xy + wh), 1)
    scores = rng.uniform(0, 1, n)
    kept = KO.nms(boxes, scores, 0.45)

    def iou(a, b):
        iw = max(0.0, min(a[2], b[2]) - max(a[0], b[0]))
        ih = max(0.0, min(a[3], b[3]) - max(a[1], b[1]))
        inter = iw * ih
        return inter / ((a[2] - a[0]) * (a[3] - a[1]) + (b[2] - b[0]) * (b[3] - b[1]) - inter)

    rank = {int(i): r for r, i in enumerate(np.argsort(-scores, kind='stable'))}
    ks = set(kept)
    for i in range(n):
        if i in ks:
            assert all(iou(boxes[i], boxes[j]) <= 0.45 for j in kept if j != i)
        else:
            assert any(iou(boxes[i], boxes[j]) > 0.45 and rank[j] < rank[i] for j in kept)
    assert [rank[i] for i in kept] == sorted(rank[i] for i in kept)


def test_kadc4_state_dict_loads_into_kadconv():
    """Checkpoint interop (KAD-Conv/README.md:39-55): a KAD-CNet KADC4_m layer's state dict
    loads strictly into kadconv.KADConv of the same width and hidden size, and both modules
    then compute the same plain forward."""
    import kadconv
    from kadcnet.kadc import KADC4_m
    torch.manual_seed(3)
    src = KADC4_m(48).eval()
    dst = kadconv.KADConv(48, se_min_hidden=64).eval()
    assert dst.load_state_dict(src.state_dict(), strict=True).missing_keys == []
    x = torch.randn(1, 48, 12, 10, generator=torch.Generator().manual_seed(4))
    with torch.no_grad():
        assert torch.equal(src(x), dst(x))
