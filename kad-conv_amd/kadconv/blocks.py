"""The other fused blocks on the north-star path.

* ``Conv1x1SiLU`` -- KAD-CNet's ``Conv`` (1x1 conv + BN + SiLU) after Conv-BN
  fusion (KAD-CNet/models/common.py:43-57, utils/torch_utils.py:244-265):
  SiLU(W x + b) as one MFMA GEMM with a fused epilogue.
* ``SqueezeExcitation`` -- the channel attention KADConv applies per branch
  (KAD-Conv/kadconv/kad_conv.py:105-109,117), as a standalone block with a
  reduction ratio: GAP -> Linear -> ReLU -> Linear -> sigmoid -> channel scale.
* ``KADDown`` -- stride-2 multi-branch downsampling with a learnable softmax
  over branches and a per-channel sigmoid selection gate.  The reference has
  no such operator; it is defined here from KADConv's branch structure
  (kad_conv.py:112-121) as
      y = sigmoid(gate) * sum_i softmax(alpha)_i * up(conv1x1_i(avgpool(x, 2^(i+1))))
  with up = bilinear (align_corners=False) to (H // 2, W // 2).

Eval-mode GPU inputs run the HIP kernels (no fallback: a missing library
raises); training mode or CPU inputs run the plain torch composition.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _ext, ops


def _use_hip(module, x):
    return (not module.training and x.is_cuda and x.dim() == 4
            and x.dtype in (torch.float32, torch.float16, torch.bfloat16))


class Conv1x1SiLU(nn.Module):
    def __init__(self, c1, c2):
        super().__init__()
        self.conv = nn.Conv2d(c1, c2, 1, bias=True)
        self._packed = {}

    @classmethod
    def from_conv_bn(cls, conv, bn):
        """Fold a bias-free 1x1 Conv2d followed by BatchNorm2d (eval statistics)."""
        m = cls(conv.in_channels, conv.out_channels)
        with torch.no_grad():
            a = bn.weight / torch.sqrt(bn.running_var + bn.eps)
            m.conv.weight.copy_(conv.weight * a.view(-1, 1, 1, 1))
            b = conv.bias if conv.bias is not None else torch.zeros_like(bn.bias)
            m.conv.bias.copy_((b - bn.running_mean) * a + bn.bias)
        return m.to(conv.weight.device)

    def forward(self, x):
        if _use_hip(self, x):
            # packed weights and the fp32 bias are cached per parameter version
            key = (x.dtype, self.conv.weight._version, self.conv.weight.data_ptr(), self.conv.bias._version,
                   self.conv.bias.data_ptr())
            if key not in self._packed:
                self._packed = {key: (_ext.gemm_pack_weights(self.conv.weight, x.dtype),
                                      self.conv.bias.detach().float().contiguous())}
            wpack, bias = self._packed[key]
            with torch.no_grad():
                return ops.conv1x1(x, self.conv.weight, bias, act='silu', wpack=wpack)
        return F.silu(self.conv(x))


class SqueezeExcitation(nn.Module):
    def __init__(self, c, reduction=16, min_hidden=1):
        super().__init__()
        hid = max(min_hidden, c // reduction)
        self.fc = nn.Sequential(nn.Linear(c, hid), nn.ReLU(), nn.Linear(hid, c), nn.Sigmoid())
        self._f32 = {}

    def forward(self, x):
        if _use_hip(self, x):
            # fp32 copies of the MLP parameters, cached per parameter version
            ps = (self.fc[0].weight, self.fc[0].bias, self.fc[2].weight, self.fc[2].bias)
            key = tuple((p._version, p.data_ptr()) for p in ps)
            if key not in self._f32:
                self._f32 = {key: tuple(p.detach().float().contiguous() for p in ps)}
            with torch.no_grad():
                return ops.squeeze_excitation(x, *self._f32[key])
        return x * self.fc(x.mean(dim=(2, 3))).view(x.shape[0], -1, 1, 1)


class KADDown(nn.Module):
    def __init__(self, c1, c2, n=3):
        super().__init__()
        self.n = n
        self.proj = nn.ModuleList(nn.Conv2d(c1, c2, 1) for _ in range(n))
        self.alpha = nn.Parameter(torch.zeros(n))
        self.gate = nn.Parameter(torch.zeros(c2))
        self._packed = {}

    def _plain(self, x):
        ho, wo = x.shape[2] // 2, x.shape[3] // 2
        a = torch.softmax(self.alpha, dim=0)
        z = 0
        for i in range(self.n):
            b = self.proj[i](F.avg_pool2d(x, kernel_size=2 ** (i + 1)))
            if b.shape[2:] != (ho, wo):
                b = F.interpolate(b, size=(ho, wo), mode='bilinear', align_corners=False)
            z = z + a[i] * b
        return z * torch.sigmoid(self.gate).view(1, -1, 1, 1)

    # kad_kaddown_prep keeps a plane's 2x2, 4x4 and 8x8 means in LDS as fp32 (160 KB per CU)
    _PREP_LDS = 160 * 1024

    def _hip_eligible(self, x):
        H, W = x.shape[2:]
        pools = (H // 2) * (W // 2) + (H // 4) * (W // 4) + (H // 8) * (W // 8)
        return (_use_hip(self, x) and 1 <= self.n <= 3 and H >= 2 ** self.n and W >= 2 ** self.n
                and 4 * pools <= self._PREP_LDS)

    def forward(self, x):
        # inputs the one-pass kernel does not cover (n > 3 branches, planes whose pools exceed
        # its LDS staging, images smaller than the deepest pool) take the plain composition
        if not self._hip_eligible(x):
            return self._plain(x)
        with torch.no_grad():
            return self._fast(x)

    def _fast(self, x):
        """One input pass (kad_kaddown_prep: the pooled inputs of every branch at
        (H/2, W/2), stacked along channels) and one 1x1 GEMM over them with the
        branch projections stacked along Cin; softmax(alpha) and sigmoid(gate)
        are folded into the packed weights and bias.  A 1x1 projection commutes
        with the bilinear resize (its weights sum to 1), so this equals the
        per-branch form of ``_plain``."""
        N, C, H, W = x.shape
        c2 = self.proj[0].weight.shape[0]
        dtype = x.dtype
        # folded weights are cached per parameter version (no per-call host work)
        params = [p.weight for p in self.proj] + [p.bias for p in self.proj] + [self.alpha, self.gate]
        key = (dtype,) + tuple((p._version, p.data_ptr()) for p in params)
        if key not in self._packed:
            a = torch.softmax(self.alpha.detach().float(), dim=0)
            g = torch.sigmoid(self.gate.detach().float())
            w = torch.cat([a[i] * self.proj[i].weight.detach().float().reshape(c2, C) for i in range(self.n)], dim=1)
            b = sum(a[i] * self.proj[i].bias.detach().float() for i in range(self.n))
            self._packed = {key: (_ext.gemm_pack_weights(w * g[:, None], dtype), (g * b).contiguous())}
        wpack, bias = self._packed[key]
        if N == 0:  # nothing to compute: the empty result
            return torch.empty(N, c2, H // 2, W // 2, dtype=dtype, device=x.device)
        u = torch.empty(N, self.n * C, H // 2, W // 2, dtype=dtype, device=x.device)
        _ext.kaddown_prep(x.contiguous(), u, self.n)
        out = torch.empty(N, c2, H // 2, W // 2, dtype=dtype, device=x.device)
        _ext.gemm1x1_fwd(u, _ext.KAD_NCHW, self.n * C, wpack, c2, out, _ext.KAD_NCHW, bias=bias)
        if x.is_contiguous(memory_format=torch.channels_last) and not x.is_contiguous():
            out = out.contiguous(memory_format=torch.channels_last)
        return out
