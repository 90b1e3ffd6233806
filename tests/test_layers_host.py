"""Host-side logic of the CCQ layers that needs no GPU: the recurrent-cache tuple forms, attention-mask
unpadding, and the short causal convolution with its cache and varlen restarts."""

import torch

D = torch.float64


def test_cache_tuple_forms():
    # the reference accepts 4-, 3- and 2-tuples (ccq/gdn/layer.py:318-336)
    from ccq_amd.layers import unpack_recurrent_state
    assert unpack_recurrent_state(("S", "C", "m", 7)) == ("S", "C", "m", 7)
    assert unpack_recurrent_state(("S", "C", 5)) == ("S", "C", None, 5)
    assert unpack_recurrent_state(("S", "C")) == ("S", "C", None, 0)
    assert unpack_recurrent_state(None) == (None, None, None, 0)


def test_unpad_and_pad_roundtrip():
    from ccq_amd.layers import get_unpad_data, index_first_axis, pad_input
    mask = torch.tensor([[1, 1, 1, 1], [0, 0, 1, 1], [0, 1, 1, 1]])
    x = torch.arange(3 * 4 * 2, dtype=D).view(3, 4, 2)
    idx, cu, mx = get_unpad_data(mask)
    assert cu.tolist() == [0, 4, 6, 9] and mx == 4
    packed = index_first_axis(x.reshape(-1, 2), idx)
    back = pad_input(packed, idx, 3, 4)
    assert torch.equal(back[mask.bool()], x[mask.bool()]) and torch.count_nonzero(back[~mask.bool()]) == 0


def test_short_convolution_cache_and_varlen():
    # causal depthwise conv: one pass == prefix pass + continuation from the cache; varlen ==
    # separate sequences
    from ccq_amd.layers import ShortConvolution
    torch.manual_seed(0)
    conv = ShortConvolution(8, 4).double()
    x = torch.randn(2, 20, 8, dtype=D)
    full, _ = conv(x)
    a, st = conv(x[:, :13], output_final_state=True)
    b, _ = conv(x[:, 13:], cache=st)
    assert torch.allclose(torch.cat([a, b], 1), full)
    cu = torch.tensor([0, 20, 40])
    pk, _ = conv(x.reshape(1, 40, 8), cu_seqlens=cu)
    assert torch.allclose(pk.view(2, 20, 8), full)


def test_conv_cache_width_w_is_accepted():
    # a cache holding the last W inputs gives the same result as one holding the last W - 1
    import torch
    from ccq_amd.layers import ShortConvolution
    torch.manual_seed(0)
    m = ShortConvolution(16, 4, bias=False, activation='silu').double()
    x = torch.randn(2, 5, 16, dtype=torch.float64)
    full = torch.randn(2, 16, 4, dtype=torch.float64)
    y_w, c_w = m(x, full, True)
    y_w1, c_w1 = m(x, full[..., 1:], True)
    assert torch.equal(y_w, y_w1) and torch.equal(c_w, c_w1) and c_w.shape == (2, 16, 3)
    import pytest
    with pytest.raises(ValueError):
        m(x, full[..., :2], True)
