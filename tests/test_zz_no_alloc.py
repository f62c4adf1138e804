"""The allocation-free attention entry point
(svl_bidirectional_attention_noalloc, through the C ABI) against the
allocating one it varies (svl_bidirectional_attention, kernels.rs:1037-1135):
the same kernels, so the same bits, on two calls in a row with the second
smaller than the first (the per-GPU scratch keeps the first call's work items
and flag, which the second must not see). Also: a non-finite result raises
Internal and the next call starts from a clear flag, and sizes beyond the
scratch are rejected with LimitExceeded before anything runs."""
import numpy as np
import pytest
import torch

import svl_amd as S

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

# (seq, heads, kv heads, head_dim, window): a large call then a smaller one
SHAPES = [
    ((700, 3, 1, 256, 512), (37, 3, 1, 256, None)),
    ((300, 12, 12, 64, None), (64, 12, 12, 64, 16)),
    ((131, 6, 2, 128, None), (50, 6, 2, 128, 7)),
    ((33, 4, 1, 512, None), (9, 4, 1, 512, None)),
    ((21, 2, 1, 8, 2), (5, 2, 1, 8, None)),
]


def inputs(seq, nh, nkv, hd, seed):
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal(seq * nh * hd) * 0.25).astype(np.float32)
    k = (rng.standard_normal(seq * nkv * hd) * 0.25).astype(np.float32)
    v = rng.standard_normal(seq * nkv * hd).astype(np.float32)
    return [torch.from_numpy(a).to(DEV) for a in (q, k, v)]


def call(fn, shape, tensors):
    seq, nh, nkv, hd, window = shape
    out = torch.full((seq * nh * hd,), float("nan"), dtype=torch.float32, device=DEV)
    fn(*tensors, seq, nh, nkv, hd, window, 1.0, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("big,small", SHAPES)
def test_noalloc_attention_equals_the_allocating_entry_point(big, small):
    tb = inputs(*big[:4], seed=1)
    ts = inputs(*small[:4], seed=2)
    got_big = call(S.bidirectional_attention_noalloc, big, tb)
    got_small = call(S.bidirectional_attention_noalloc, small, ts)
    want_big = call(S.bidirectional_attention, big, tb)
    want_small = call(S.bidirectional_attention, small, ts)
    for got, want, label in ((got_big, want_big, big), (got_small, want_small, small)):
        assert np.isfinite(got).all(), label
        assert got.tobytes() == want.tobytes(), label


def test_noalloc_attention_flag_is_cleared_between_calls():
    shape = (40, 3, 1, 256, None)
    q, k, v = inputs(*shape[:4], seed=3)
    bad = q.clone()
    bad[5] = float("nan")
    with pytest.raises(S.SvlError) as e:
        call(S.bidirectional_attention_noalloc, shape, (bad, k, v))
    assert e.value.kind == "Internal"
    got = call(S.bidirectional_attention_noalloc, shape, (q, k, v))
    assert got.tobytes() == call(S.bidirectional_attention, shape, (q, k, v)).tobytes()


def test_noalloc_attention_rejects_sizes_beyond_its_scratch():
    # 8193 keys: above the 8192 the scratch holds (the allocating entry point
    # takes it). Real buffers of the full size, although nothing is launched.
    seq, hd = 8193, 64
    q, k, v = (torch.zeros(seq * hd, device=DEV) for _ in range(3))
    out = torch.empty(seq * hd, device=DEV)
    with pytest.raises(S.SvlError) as e:
        S.bidirectional_attention_noalloc(q, k, v, seq, 1, 1, hd, None, 1.0, out)
    assert e.value.kind == "LimitExceeded"
    # 8192 keys of 512 heads sharing one KV head: 32768 work items > 16384
    seq, nh = 8192, 512
    q = torch.zeros(seq * nh * hd, device=DEV)
    k, v = (torch.zeros(seq * hd, device=DEV) for _ in range(2))
    out = torch.empty(seq * nh * hd, device=DEV)
    with pytest.raises(S.SvlError) as e:
        S.bidirectional_attention_noalloc(q, k, v, seq, nh, 1, hd, None, 1.0, out)
    assert e.value.kind == "LimitExceeded"
    del q, out
    shape = (64, 3, 1, 256, None)
    t = inputs(*shape[:4], seed=4)
    assert call(S.bidirectional_attention_noalloc, shape, t).tobytes() == \
        call(S.bidirectional_attention, shape, t).tobytes()
