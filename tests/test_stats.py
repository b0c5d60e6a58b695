"""tda_amd.tile_sparsity: the tile-occupancy map and skip counters of one forward pass.
CPU: bit unpacking and argument checks.  GPU: the map against the oracle's weights, the
counters against the map, the output against the plain entry points."""
import pytest
import torch

from oracle.formula import tau
from tests.helpers import make_inputs


def test_unpack_bits():
    from tda_amd.stats import _unpack
    branches, b, h, t = 2, 1, 3, 37  # two words per tile row
    want = torch.rand(branches, b, h, t, t) < 0.3
    bits = torch.zeros(branches, b, h, t, 64, dtype=torch.int64)
    bits[..., :t] = want.to(torch.int64)
    words = (bits.view(branches, b, h, t, 2, 32) << torch.arange(32)).sum(-1)
    words = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    assert torch.equal(_unpack(words.flatten(), branches, b, h, t), want)


def test_argument_checks():
    from tda_amd import tile_sparsity
    x = torch.randn(1, 2, 40, 64)
    with pytest.raises(ValueError, match="GPU"):
        tile_sparsity(x, x, x, 1.0)
    with pytest.raises(ValueError, match="q2, k2 and lambda_param"):
        tile_sparsity(x, x, x, 1.0, q2=x)


def _tile_map(q, k, n, d, beta, normalize, floor=0.0):
    """Tiles holding a weight with x > floor (floor > 0: weights clear of rounding ties)."""
    qf, kf = q.double().cpu(), k.double().cpu()
    if normalize:
        qf = torch.nn.functional.normalize(qf, dim=-1)
        kf = torch.nn.functional.normalize(kf, dim=-1)
    s = qf @ kf.transpose(-1, -2) - tau(n, d, beta)[:, None]
    nz = (s > floor) & torch.ones(n, n, dtype=torch.bool).tril()
    t = (n + 31) // 32
    pad = torch.zeros(*nz.shape[:-2], 32 * t, 32 * t, dtype=torch.bool)
    pad[..., :n, :n] = nz
    return pad.view(*nz.shape[:-2], t, 32, t, 32).any(-1).any(-2)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tile_sparsity_tda(dtype):
    from tda_amd import differential_threshold_rela_triton, tile_sparsity
    shape = (2, 3, 700, 128)
    q1, q2, k1, k2, v = make_inputs(shape, 11, 5, dtype)
    out, st = tile_sparsity(q1, k1, v, 1.0, 2.0, True, q2=q2, k2=k2, lambda_param=0.5)
    ref = differential_threshold_rela_triton(q1, q2, k1, k2, v, 1.0, 0.5, 2.0, True)
    assert torch.equal(out, ref)
    t = (700 + 31) // 32
    assert st.occupancy.shape == (2, 2, 3, t, t)
    assert st.tiles_causal == 2 * 2 * 3 * t * (t + 1) // 2
    assert st.tiles_nonzero == int(st.occupancy.sum())
    assert not st.occupancy.triu(1).any()
    want = torch.stack([_tile_map(q1, k1, 700, 128, 1.0, True), _tile_map(q2, k2, 700, 128, 1.0, True)])
    mism = (st.occupancy.cpu() != want).sum().item()
    assert mism <= 4, mism  # threshold ties within rounding only
    # one-sided: every tile with a weight clear of rounding ties is in the map
    strong = torch.stack([_tile_map(q1, k1, 700, 128, 1.0, True, 4e-6), _tile_map(q2, k2, 700, 128, 1.0, True, 4e-6)])
    assert not (strong & ~st.occupancy.cpu()).any()
    assert 0.0 < st.skipped_fraction < 1.0
    assert st.density.shape == (2,)
    # normalised with more than one query tile: both dtypes run the int8 screen first
    assert st.tiles_screened >= st.tiles_nonzero


@pytest.mark.gpu
def test_tile_sparsity_tra_unnormalized():
    from tda_amd import threshold_rela_triton, tile_sparsity
    q, k, v = make_inputs((1, 2, 300, 64), 12, 3, torch.bfloat16)
    out, st = tile_sparsity(q, k, v, 25.0, 1.0)
    assert torch.equal(out, threshold_rela_triton(q, k, v, 25.0, 1.0))
    # no screen without normalisation: the block tile pass scores all 2 x 55 causal tiles
    assert st.tiles_causal == 2 * 10 * 11 // 2 and st.tiles_screened is None
    assert st.tiles_nonzero == int(st.occupancy.sum())
    want = _tile_map(q, k, 300, 64, 25.0, False).unsqueeze(0)
    assert (st.occupancy.cpu() != want).sum().item() <= 4
    strong = _tile_map(q, k, 300, 64, 25.0, False, 1e-4).unsqueeze(0)
    assert not (strong & ~st.occupancy.cpu()).any()
    assert st.tiles_nonzero == int(st.occupancy.sum())
