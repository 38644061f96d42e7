"""Host-side pieces of the encoder model that need no GPU."""

import torch
import torch.nn.functional as F

from trifusion_amd.model import FFN_ALIGN, Encoder, ModelConfig


def _swiglu(x):
    g, u = x.chunk(2, -1)
    return F.silu(g) * u


def test_padded_ffn_weights_give_the_same_ffn():
    """Each FFN half padded with zero rows (and down with zero columns) to a
    multiple of FFN_ALIGN: same result as the 1365-wide FFN up to summation order."""
    torch.manual_seed(0)
    blk = Encoder(ModelConfig(depth=1)).eval().blocks[0]
    g1, g2 = blk._padded_ffn()
    f = blk.down.in_features
    fp = g2.shape[1]
    assert fp % FFN_ALIGN == 0 and fp >= f and g1.shape == (2 * fp, blk.down.out_features)
    assert torch.equal(g1[:f], blk.gate_up.weight[:f]) and torch.equal(g1[fp : fp + f], blk.gate_up.weight[f:])
    assert not g1[f:fp].any() and not g1[fp + f :].any() and not g2[:, f:].any()
    h = torch.randn(3, 7, blk.down.out_features)
    ref = F.linear(_swiglu(F.linear(h, blk.gate_up.weight)), blk.down.weight)
    pad = F.linear(_swiglu(F.linear(h, g1)), g2)
    assert (ref - pad).abs().max() <= 1e-6 * ref.abs().max()


def test_padded_ffn_rebuilt_when_weights_change():
    torch.manual_seed(1)
    blk = Encoder(ModelConfig(depth=1)).eval().blocks[0]
    first = blk._padded_ffn()
    assert blk._padded_ffn() is first
    with torch.no_grad():
        blk.down.weight.mul_(2)
    second = blk._padded_ffn()
    assert second is not first and torch.equal(second[1][:, : blk.down.in_features], blk.down.weight)
