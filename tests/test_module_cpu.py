"""Drop-in surface of the module, checked without a GPU: constructor, attribute
names, parameter names/shapes/order and default init match the reference
(infinity/video/attention.py:34-80), so reference state_dicts load unchanged."""

import copy

import pytest
import torch

from goldens import CASES, load, regenerate
from megaslide_amd import DeformableSlideAttention3D
from oracle.dsa3d_ref import PARAM_NAMES, param_shapes


@pytest.mark.parametrize("D,nh,kernel", [(16, 2, (3, 7, 7)), (24, 3, (3, 5, 5)), (8, 2, (1, 3, 3)),
                                         (1024, 16, (3, 7, 7))])
def test_parameter_names_shapes_order(D, nh, kernel):
    m = DeformableSlideAttention3D(D, nh, kernel_size=kernel)
    names = [n for n, _ in m.named_parameters()]
    assert tuple(names) == PARAM_NAMES
    shapes = param_shapes(D, nh, kernel)
    for n, p in m.named_parameters():
        assert tuple(p.shape) == shapes[n], n
    assert torch.count_nonzero(m.offset_net[-1].weight) == 0
    assert torch.count_nonzero(m.offset_net[-1].bias) == 0
    assert (m.hidden_size, m.num_heads, m.head_dim) == (D, nh, D // nh)
    assert (m.k_t, m.k_h, m.k_w) == tuple(kernel)
    assert isinstance(m.offset_net, torch.nn.Sequential) and len(m.offset_net) == 3
    assert isinstance(m.offset_net[1], torch.nn.GELU)


def test_defaults_and_deepcopy():
    m = DeformableSlideAttention3D(32, 4)
    assert (m.k_t, m.k_h, m.k_w) == (3, 7, 7)
    assert m.offset_scale == 1.0 and m.dropout.p == 0.0
    m2 = copy.deepcopy(m)
    for (n1, p1), (n2, p2) in zip(m.named_parameters(), m2.named_parameters()):
        assert n1 == n2 and torch.equal(p1, p2)


@pytest.mark.parametrize("name", [c["name"] for c in CASES if c["mode"] == "net"])
def test_reference_state_dict_loads(name):
    meta, _ = load(name)
    case, p, *_ = regenerate(meta)
    m = DeformableSlideAttention3D(case["D"], case["nh"], kernel_size=tuple(case["kernel"]),
                                   offset_scale=case["scale"]).double()
    sd = {k: torch.from_numpy(v) for k, v in p.items()}
    missing, unexpected = m.load_state_dict(sd, strict=True)
    assert not missing and not unexpected
    assert list(m.state_dict().keys()) == meta["param_names"]


class _Config:
    """The MegaSlideConfig fields a DiTBlock reads (infinity/video/config.py)."""

    def __init__(self, hidden_size, num_heads, dsa_kernel_size=(3, 7, 7), offset_scale=1.0,
                 dropout=0.0, mlp_ratio=4.0, use_text_conditioning=False):
        self.hidden_size, self.num_heads = hidden_size, num_heads
        self.dsa_kernel_size, self.offset_scale, self.dropout = dsa_kernel_size, offset_scale, dropout
        self.mlp_ratio, self.use_text_conditioning = mlp_ratio, use_text_conditioning

    @property
    def mlp_hidden_size(self):
        return int(self.hidden_size * self.mlp_ratio)


def test_dit_block_parameters_match_reference_block():
    """The drop-in DiTBlock registers the reference block's parameters in its
    order (the golden fixture records the reference's named_parameters()), with
    the same shapes, and loads the reference's values strictly."""
    from inputs import BLOCK, block_params
    from megaslide_amd import DiTBlock

    meta, arrs = load(BLOCK["name"])
    cfg = _Config(BLOCK["D"], BLOCK["nh"], BLOCK["kernel"], BLOCK["scale"],
                  mlp_ratio=BLOCK["mlp_ratio"])
    blk = DiTBlock(cfg)
    assert [n for n, _ in blk.named_parameters()] == meta["param_names"]
    p = block_params(BLOCK)
    sd = {n: torch.from_numpy(v).float() for n, v in p.items()}
    blk.load_state_dict(sd, strict=True)
    for n, prm in blk.named_parameters():
        assert prm.shape == tuple(arrs["grad." + n].shape), n
    # text conditioning adds the reference's norm_cross and cross_attn, in order
    names = [n for n, _ in DiTBlock(_Config(32, 2, use_text_conditioning=True)).named_parameters()]
    assert names[-6:] == ["norm_cross.weight", "norm_cross.bias", "cross_attn.in_proj_weight",
                          "cross_attn.in_proj_bias", "cross_attn.out_proj.weight",
                          "cross_attn.out_proj.bias"]
