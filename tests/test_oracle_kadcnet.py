"""Closed-form pins of the KAD-CNet oracle's blocks (oracle/kadcnet_oracle.py), written
from the reference's documented compositions, with no module of this package:

  ELAN1 (KAD-CNet/models/common.py:580-598)      cv1 split in halves, cv2 and cv3 chained
                                                  on the second, cat(y0, y1, y2, y3), cv4
  RepNCSP_KADC (models/module/KADC/module.py:74-89)  cv3(cat(m(cv1(x)), cv2(x)))
  RepNCSPELAN4_KADC (module.py:92-111)            the ELAN1 chain with (RepNCSP, 3x3 Conv) stages
  SPPELAN (common.py:563-577)                     cv1, three chained 5x5 / stride-1 max pools,
                                                  cat of all four, cv5
  AConv (common.py:60-67)                         2x2 / stride-1 average pool, 3x3 / stride-2 Conv
  DDetect heads (models/yolo.py:102-105)          cat(cv2 box branch, cv3 class branch), the box
                                                  branch's last 1x1 conv in 4 groups
  non_max_suppression (utils/general.py:881-990)  confidence filter, best class, class-offset
                                                  boxes (7680 px a class), greedy IoU, max_det

Every convolution is a fused one (``conv.weight`` + ``conv.bias``, then SiLU) whose weights
are channel selectors or centre-tap identities with distinct gains, so each block's output
is a closed form of the input computed here with numpy: a swapped half, a wrong chain input,
a permuted concat, a wrong pool window, stride or padding, or a wrong group map each change
the result well beyond the 1e-12 bound."""
import numpy as np
import torch

from oracle import kadcnet_oracle as O
from oracle import kadconv_oracle as K
from kadconv import synthetic as S


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _sig(v):
    return 1.0 / (1.0 + np.exp(-v))


def _sel(rows, cin, gains=None, k=1):
    """Fused-conv weight [len(rows), cin, k, k]: output o reads input rows[o] at the centre tap."""
    w = torch.zeros(len(rows), cin, k, k, dtype=torch.float64)
    for o, r in enumerate(rows):
        w[o, r, k // 2, k // 2] = 1.0 if gains is None else gains[o]
    return w


def _put(sd, p, w, b=None):
    sd[p + 'conv.weight'] = w
    sd[p + 'conv.bias'] = torch.zeros(w.shape[0], dtype=torch.float64) if b is None else b


def _x(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def test_elan1_chunk_chain_and_concat_order():
    c1, c3, c4, c2 = 4, 4, 2, 8
    sd, p = {}, 'b.'
    _put(sd, p + 'cv1.', _sel([0, 1, 2, 3], c1))                     # silu(x), split 2 | 2
    _put(sd, p + 'cv2.', _sel([0, 1], c3 // 2, [1.5, 0.5], k=3))     # on the second half
    _put(sd, p + 'cv3.', _sel([1, 0], c4, [2.0, 3.0], k=3))          # on cv2's output, swapped
    perm = [5, 2, 7, 0, 4, 1, 6, 3]
    b4 = torch.linspace(-0.3, 0.4, c2, dtype=torch.float64)
    _put(sd, p + 'cv4.', _sel(perm, c3 + 2 * c4), b4)
    x = _x((2, c1, 6, 5), 1)
    got = O._gelan(sd, p, x, kadc=False).numpy()
    xn = x.numpy()
    y0, y1 = _silu(xn[:, 0:2]), _silu(xn[:, 2:4])
    y2 = _silu(np.stack((1.5 * y1[:, 0], 0.5 * y1[:, 1]), 1))
    y3 = _silu(np.stack((2.0 * y2[:, 1], 3.0 * y2[:, 0]), 1))
    cat = np.concatenate((y0, y1, y2, y3), 1)
    ref = _silu(cat[:, perm] + b4.numpy()[None, :, None, None])
    assert np.abs(got - ref).max() <= 1e-12


def _zero_dsc_kadconv(dim, seed):
    """A KADConv state whose DSC weights are 0: the layer maps z to cat_i(v_i att_i) + z with
    per-channel constants v_i = scale_i relu(bn_i(dsc bias_i)) and att_i = sigmoid(W2 relu(W1 v_i
    + b1) + b2) (the mean of a constant map is the constant; its upsample is the same constant)."""
    sd = S.make_kadconv_state(dim, seed=seed, dtype=torch.float64)
    consts = []
    for i, c in enumerate(K.branch_widths(dim)):
        sd[f'convs.{i}.1.weight'].zero_()
        q = f'convs.{i}.'
        n = lambda k: sd[k].numpy().reshape(-1)  # noqa: E731
        t = (n(q + '1.bias') - n(q + '2.running_mean')) / np.sqrt(n(q + '2.running_var') + 1e-3) \
            * n(q + '2.weight') + n(q + '2.bias')
        v = np.maximum(t, 0.0) * n(f'weight.{i}.0.weight')
        hdn = np.maximum(sd[f'fc.{i}.0.weight'].numpy() @ v + n(f'fc.{i}.0.bias'), 0.0)
        consts.append(v * _sig(sd[f'fc.{i}.2.weight'].numpy() @ hdn + n(f'fc.{i}.2.bias')))
    return sd, np.concatenate(consts)


def _repncsp_state(sd, p, c1, c_, c2, n_kadc, seed):
    _put(sd, p + 'cv1.', _sel(list(range(c_)), c1, [1.0 + 0.25 * j for j in range(c_)]))
    _put(sd, p + 'cv2.', _sel([c1 - 1 - j for j in range(c_)], c1, [-0.5 - 0.1 * j for j in range(c_)]))
    perm = list(np.random.default_rng(seed).permutation(2 * c_))[:c2]
    _put(sd, p + 'cv3.', _sel(perm, 2 * c_), torch.linspace(-0.2, 0.2, c2, dtype=torch.float64))
    add = np.zeros(c_)
    for j in range(n_kadc):
        m, cst = _zero_dsc_kadconv(c_, seed + j)
        for k, v in m.items():
            sd[f'{p}m.{j}.{k}'] = v
        add = add + cst
    return perm, add


def _repncsp_ref(x, c1, c_, perm, add, b3):
    a = _silu(np.stack([(1.0 + 0.25 * j) * x[:, j] for j in range(c_)], 1)) + add[None, :, None, None]
    c = _silu(np.stack([(-0.5 - 0.1 * j) * x[:, c1 - 1 - j] for j in range(c_)], 1))
    return _silu(np.concatenate((a, c), 1)[:, perm] + b3[None, :, None, None])


def test_repncsp_concat_order_and_kadconv_on_the_cv1_branch():
    c1, c_, c2 = 6, 6, 10
    x = _x((2, c1, 7, 9), 2)
    for n_kadc in (0, 2):
        sd, p = {}, 'r.'
        perm, add = _repncsp_state(sd, p, c1, c_, c2, n_kadc, seed=3)
        got = O._repncsp(sd, p, x).numpy()
        ref = _repncsp_ref(x.numpy(), c1, c_, perm, add, sd[p + 'cv3.conv.bias'].numpy())
        assert np.abs(got - ref).max() <= 1e-12, (n_kadc, np.abs(got - ref).max())


def test_repncspelan4_kadc_stage_chain():
    """RepNCSPELAN4_KADC: y0 | y1 = halves of cv1(x); y2 = cv2.1(RepNCSP cv2.0(y1)); y3 =
    cv3.1(RepNCSP cv3.0(y2)); cv4(cat(y0, y1, y2, y3))."""
    c1, c3, c4, c2 = 6, 12, 6, 9
    sd, p = {}, 'g.'
    _put(sd, p + 'cv1.', _sel(list(range(c1)) * 2, c1, [1.0] * c1 + [0.5] * c1))
    parts = []
    for stage, cin, seed in (('cv2.', c3 // 2, 5), ('cv3.', c4, 7)):
        parts.append(_repncsp_state(sd, p + stage + '0.', cin, c4, c4, 1, seed))
        _put(sd, p + stage + '1.', _sel(list(range(c4))[::-1], c4, [0.7] * c4, k=3))
    perm4 = list(np.random.default_rng(9).permutation(c3 + 2 * c4))[:c2]
    _put(sd, p + 'cv4.', _sel(perm4, c3 + 2 * c4), torch.linspace(0.1, -0.1, c2, dtype=torch.float64))
    x = _x((1, c1, 5, 8), 4)
    got = O._gelan(sd, p, x, kadc=True).numpy()
    xn = x.numpy()
    y0, y1 = _silu(xn), _silu(0.5 * xn)
    ys = [y0, y1]
    for (perm, add), st in zip(parts, ('cv2.', 'cv3.')):
        t = _repncsp_ref(ys[-1], ys[-1].shape[1], c4, perm, add, sd[p + st + '0.cv3.conv.bias'].numpy())
        ys.append(_silu(0.7 * t[:, ::-1]))
    ref = _silu(np.concatenate(ys, 1)[:, perm4] + sd[p + 'cv4.conv.bias'].numpy()[None, :, None, None])
    assert np.abs(got - ref).max() <= 1e-12


def test_sppelan_single_peaks_give_squares_of_side_1_5_9_13():
    """One positive peak per channel: silu is increasing on [0, inf), so the three chained
    5x5 max pools (stride 1, padding 2) of silu(x) are the peak's value on squares of side 5,
    9 and 13 around it, clipped at the border; cv5 permutes the four maps' channels."""
    c1, c3, c2, H, W = 2, 2, 8, 18, 20
    sd, p = {}, 's.'
    _put(sd, p + 'cv1.', _sel([0, 1], c1))
    perm = [6, 1, 3, 4, 0, 7, 2, 5]
    _put(sd, p + 'cv5.', _sel(perm, 4 * c3), torch.linspace(-0.1, 0.3, c2, dtype=torch.float64))
    x = torch.zeros(1, c1, H, W, dtype=torch.float64)
    peaks = [(9, 8, 1.3), (1, 18, 2.1)]                      # the second one near a corner
    for c, (r, q, v) in enumerate(peaks):
        x[0, c, r, q] = v
    got = O._sppelan(sd, p, x).numpy()
    maps = []
    for k in range(4):
        m = np.zeros((c1, H, W))
        for c, (r, q, v) in enumerate(peaks):
            m[c, max(r - 2 * k, 0):r + 2 * k + 1, max(q - 2 * k, 0):q + 2 * k + 1] = _silu(v)
        maps.append(m)
    ref = _silu(np.concatenate(maps, 0)[perm] + sd[p + 'cv5.conv.bias'].numpy()[:, None, None])[None]
    assert np.abs(got - ref).max() <= 1e-12


def test_aconv_on_a_ramp():
    """avg_pool2d(2, stride 1, no padding) of x = a + b h + d w is the line at (h + 0.5, w + 0.5)
    on an (H - 1) x (W - 1) grid; the 3x3 stride-2 Conv (padding 1) with a centre-tap weight reads
    its pixel (2 j, 2 k): the output is silu(g (a + b (2 j + 0.5) + d (2 k + 0.5)) + beta)."""
    c, H, W = 3, 12, 15
    sd, p = {}, 'a.'
    gains = [0.8, -1.2, 0.5]
    beta = torch.tensor([0.1, -0.2, 0.05], dtype=torch.float64)
    _put(sd, p + 'cv1.', _sel([0, 1, 2], c, gains, k=3), beta)
    g = torch.Generator().manual_seed(6)
    a = torch.rand(c, generator=g, dtype=torch.float64)
    b = torch.rand(c, generator=g, dtype=torch.float64) * 0.2
    d = torch.rand(c, generator=g, dtype=torch.float64) * 0.2 - 0.1
    hh = torch.arange(H, dtype=torch.float64).view(1, H, 1)
    ww = torch.arange(W, dtype=torch.float64).view(1, 1, W)
    x = (a.view(c, 1, 1) + b.view(c, 1, 1) * hh + d.view(c, 1, 1) * ww).unsqueeze(0)
    got = O._aconv(sd, p, x).numpy()[0]
    ho, wo = (H - 1 + 2 - 3) // 2 + 1, (W - 1 + 2 - 3) // 2 + 1
    jj = 2 * np.arange(ho)[:, None] + 0.5
    kk = 2 * np.arange(wo)[None, :] + 0.5
    ref = np.stack([_silu(gains[i] * (a[i].item() + b[i].item() * jj + d[i].item() * kk) + beta[i].item())
                    for i in range(c)])
    assert got.shape == ref.shape
    assert np.abs(got - ref).max() <= 1e-12


def test_ddetect_heads_concat_order_and_box_groups():
    """Zero weights before the last 1x1 convs make their inputs the constants silu(beta); the
    box conv (4 groups of c2 / 4 inputs) then gives W[o] . silu(beta1[group(o)]) + b[o], the
    class conv Wc silu(betac) + bc, and the head map is cat(box, class) at every pixel."""
    nc, c2, c3, cin = 5, 64, 12, 7
    sd, p = {}, 'd.'
    g = torch.Generator().manual_seed(8)
    rnd = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    consts = {}
    for br, cc in (('cv2', c2), ('cv3', c3)):
        for j in (0, 1):
            q = f'{p}{br}.0.{j}.'
            groups = 4 if (br == 'cv2' and j == 1) else 1
            w = torch.zeros(cc, (cin if j == 0 else cc) // groups, 3, 3, dtype=torch.float64)
            beta = rnd(cc)
            _put(sd, q, w, beta)
            consts[(br, j)] = _silu(beta.numpy())
    wb, bb = rnd(4 * 16, c2 // 4, 1, 1), rnd(4 * 16)
    wc, bc = rnd(nc, c3, 1, 1), rnd(nc)
    sd[f'{p}cv2.0.2.weight'], sd[f'{p}cv2.0.2.bias'] = wb, bb
    sd[f'{p}cv3.0.2.weight'], sd[f'{p}cv3.0.2.bias'] = wc, bc
    x = _x((2, cin, 4, 6), 9)
    got = O.ddetect_heads(sd, p, [x], nc)[0].numpy()
    s1 = consts[('cv2', 1)]
    box = np.array([wb[o, :, 0, 0].numpy() @ s1[(o // 16) * (c2 // 4):(o // 16 + 1) * (c2 // 4)] + bb[o].item()
                    for o in range(64)])
    cls = wc[:, :, 0, 0].numpy() @ consts[('cv3', 1)] + bc.numpy()
    ref = np.concatenate((box, cls))[None, :, None, None] * np.ones((2, 1, 4, 6))
    assert got.shape == (2, 64 + nc, 4, 6)
    assert np.abs(got - ref).max() <= 1e-12


def _pred(rows, nc):
    """[1, 4 + nc, A] prediction from (cx, cy, w, h, class scores) rows."""
    a = np.array([list(r[:4]) + list(r[4]) for r in rows], dtype=np.float64)
    assert a.shape[1] == 4 + nc
    return torch.from_numpy(a.T[None].copy())


def test_non_max_suppression_known_answers():
    rows = [
        (50, 50, 20, 20, (0.9, 0.1, 0.0)),    # 0: kept
        (50, 50, 20, 20, (0.0, 0.8, 0.1)),    # 1: same box, other class: kept (class offset)
        (52, 50, 20, 20, (0.7, 0.0, 0.2)),    # 2: IoU 0.82 with 0, same class: suppressed
        (200, 200, 10, 10, (0.1, 0.1, 0.2)),  # 3: best score 0.2 < conf 0.25: filtered
        (300, 300, 10, 10, (0.0, 0.3, 0.6)),  # 4: kept (class 2)
        (52, 50, 20, 20, (0.05, 0.5, 0.3)),   # 5: best class 1, IoU 0.82 with 1: suppressed
    ]
    pred = _pred(rows, 3)

    def ids(out):
        o = out[0].numpy()
        return [(round(float(r[4]), 6), int(r[5])) for r in o], o

    got, o = ids(O.non_max_suppression(pred, conf_thres=0.25, iou_thres=0.45))
    assert got == [(0.9, 0), (0.8, 1), (0.6, 2)]
    assert np.allclose(o[0, :4], [40, 40, 60, 60]) and np.allclose(o[2, :4], [295, 295, 305, 305])
    got, _ = ids(O.non_max_suppression(pred, conf_thres=0.25, iou_thres=0.45, max_det=2))
    assert got == [(0.9, 0), (0.8, 1)]
    got, _ = ids(O.non_max_suppression(pred, conf_thres=0.25, iou_thres=0.45, agnostic=True))
    assert got == [(0.9, 0), (0.6, 2)]
    got, _ = ids(O.non_max_suppression(pred, conf_thres=0.25, iou_thres=0.9))   # IoU 0.82 < 0.9
    assert got == [(0.9, 0), (0.8, 1), (0.7, 0), (0.6, 2), (0.5, 1)]
    got, _ = ids(O.non_max_suppression(pred, conf_thres=0.65, iou_thres=0.45))
    assert got == [(0.9, 0), (0.8, 1)]
