"""Host-side pieces of the encoder model that need no GPU."""

import torch
import torch.nn.functional as F

from trifusion_amd.mamba import PROJ_ALIGN
from trifusion_amd.model import FFN_ALIGN, Encoder, ModelConfig


def _swiglu(x):
    g, u = x.chunk(2, -1)
    return F.silu(g) * u


def test_padded_ffn_weights_give_the_same_ffn():
    """Each FFN half padded with zero rows (and down with zero columns) to a
    multiple of FFN_ALIGN, gate_up stored K-major: same result as the
    1365-wide FFN up to summation order."""
    torch.manual_seed(0)
    blk = Encoder(ModelConfig(depth=1)).eval().blocks[0]
    g1t, g2 = blk._padded_ffn()
    f = blk.down.in_features
    fp = g2.shape[1]
    assert fp % FFN_ALIGN == 0 and fp >= f and g1t.shape == (blk.down.out_features, 2 * fp)
    assert g1t.is_contiguous()
    g1 = g1t.t()
    assert torch.equal(g1[:f], blk.gate_up.weight[:f]) and torch.equal(g1[fp : fp + f], blk.gate_up.weight[f:])
    assert not g1[f:fp].any() and not g1[fp + f :].any() and not g2[:, f:].any()
    h = torch.randn(3, 7, blk.down.out_features)
    ref = F.linear(_swiglu(F.linear(h, blk.gate_up.weight)), blk.down.weight)
    pad = F.linear(_swiglu(h @ g1t), g2)
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


def test_padded_in_projection_keeps_the_split():
    """The in-projection runs at a multiple of PROJ_ALIGN outputs; the extra
    rows are zero and the first columns are the reference projection."""
    torch.manual_seed(2)
    m = Encoder(ModelConfig(depth=1)).eval().blocks[0].mamba
    wp = m._padded_in_proj()
    rows = m.in_proj.out_features
    assert wp.shape[0] % PROJ_ALIGN == 0 and wp.shape[0] >= rows
    assert torch.equal(wp[:rows], m.in_proj.weight) and not wp[rows:].any()
    u = torch.randn(2, 5, m.in_proj.in_features)
    assert torch.equal(F.linear(u, wp)[..., :rows], F.linear(u, m.in_proj.weight)) or torch.allclose(
        F.linear(u, wp)[..., :rows], F.linear(u, m.in_proj.weight), rtol=1e-6, atol=1e-6
    )
    assert m._padded_in_proj() is wp
    with torch.no_grad():
        m.in_proj.weight.add_(1)
    assert m._padded_in_proj() is not wp


def test_padded_stem_weight():
    from trifusion_amd.model import STEM_ALIGN

    torch.manual_seed(3)
    enc = Encoder(ModelConfig(depth=1)).eval()
    c = enc.config
    w = enc._stem_weight()
    assert w.shape[1] % STEM_ALIGN == 0 and w.shape[1] >= c.stem_kernel
    assert torch.equal(w[:, : c.stem_kernel], enc.stem.weight.reshape(c.dim, c.stem_kernel))
    assert not w[:, c.stem_kernel :].any() and enc._stem_weight() is w


def test_weight_caches_under_inference_mode():
    """A model built and cast inside torch.inference_mode() holds inference
    tensors, which have no version counter; the derived-weight caches (padded
    projection, padded FFN, stem GEMM weight, packed convolutions) still build
    and hit."""
    from trifusion_amd.trifusion import CNNStage

    with torch.inference_mode():
        torch.manual_seed(2)
        enc = Encoder(ModelConfig(depth=1)).eval().to(torch.bfloat16)
        blk = enc.blocks[0]
        assert blk.mamba.in_proj.weight.is_inference()
        wp = blk.mamba._padded_in_proj()
        assert wp.shape[0] % PROJ_ALIGN == 0 and blk.mamba._padded_in_proj() is wp
        ffn = blk._padded_ffn()
        assert blk._padded_ffn() is ffn
        stem = enc._stem_weight()
        assert enc._stem_weight() is stem
        stage = CNNStage(8, 16, 2).to(torch.bfloat16)
        packed = stage.packed()
        assert stage.packed() is packed
