"""GPU parity at the headline throughput workload, at its full size: the
shape-A text encoder (hidden 768, 24 layers, 3 query heads sharing one KV head
of dim 256, GeGLU 1152, PLE 256, vocab 262144) with seed-0 random-init
weights, 64 rows of lengths U[64, 512] (seed 1) with ids uniform over the
vocabulary (seed 1), run exactly as the throughput path runs it: ids resident
in HBM, three row groups on three streams, Matryoshka outputs 768 / 512 / 256
/ 128 written to HBM in one call.

Rows are compared with the CPU oracle (TextModel::forward_impl,
src/model/text.rs:182-538, and truncate_and_normalize, kernels.rs:911-927)
per embedding at max-abs <= 1e-4 and cosine >= 0.99999 at every dim. The
compared rows are the first and last row of every row group plus a seeded
sample of the rest, 20 in all, so every group and every group boundary is
covered; the oracle runs them on 16 host threads."""
import numpy as np
import pytest
import torch

import svl_amd as S
import svl_synth
from oracle import oracle as O

MAX_ABS = 1e-4
MIN_COS = 0.99999
BATCH, LEN_LO, LEN_HI = 64, 64, 512
DIMS = [768, 512, 256, 128]
GROUPS = 3
SPLIT_MIN_TOKENS = 4096   # batches below this many tokens run as one group


def group_starts(offsets, groups):
    """First row of every row group: group k starts at the first row
    boundary at or past k / groups of the batch's tokens, each group keeping
    at least one row (the library's split of a batch over its streams)."""
    B, T = len(offsets) - 1, int(offsets[-1])
    ng = max(1, min(groups, B)) if T >= SPLIT_MIN_TOKENS else 1
    starts, r = [], 0
    for k in range(ng):
        starts.append(r)
        end = B
        if k + 1 < ng:
            end = max(r + 1, 1)
            while end < B - (ng - 1 - k) and ng * int(offsets[end]) < (k + 1) * T:
                end += 1
        r = end
    return starts


def cosine(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def test_group_starts_split_tokens_evenly():
    offsets = np.concatenate([[0], np.cumsum([100] * 60)])
    assert group_starts(offsets, 3) == [0, 20, 40]
    assert group_starts(np.array([0, 10, 20]), 3) == [0]   # below the split threshold
    offsets = np.concatenate([[0], np.cumsum([5000, 1, 1, 1])])
    assert group_starts(offsets, 3) == [0, 1, 2]


@pytest.mark.gpu
def test_headline_batch_matches_oracle():
    cfg = svl_synth.config_a()
    w = svl_synth.weights(cfg, seed=0)
    lengths = svl_synth.row_lengths(BATCH, LEN_LO, LEN_HI, seed=1)
    rows = svl_synth.token_rows(cfg["vocab_size"], lengths, seed=1)
    offsets = np.zeros(BATCH + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    starts = group_starts(offsets, GROUPS)
    assert len(starts) == GROUPS

    m = S.TextModel(S.TextConfig.from_json_value(cfg), w)
    m.set_stream_split(GROUPS)
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    out = torch.zeros((BATCH, sum(DIMS)), dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    m.forward_device(ids.data_ptr(), offsets, DIMS, out.data_ptr(), stream)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    # the same call again: bit-identical (text_embeddings.rs:388-397)
    m.forward_device(ids.data_ptr(), offsets, DIMS, out.data_ptr(), stream)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), got)
    m.close()

    edges = sorted({r for s in starts for r in (s - 1, s) if 0 <= r < BATCH} | {BATCH - 1})
    rest = [r for r in range(BATCH) if r not in edges]
    pick = sorted(edges + [int(r) for r in np.random.default_rng(11).choice(
        rest, 20 - len(edges), replace=False)])
    assert len(pick) == 20
    for s, e in zip(starts, starts[1:] + [BATCH]):
        assert any(s <= r < e for r in pick)
    print(f"row groups start at rows {starts}; comparing rows {pick}", flush=True)
    ref = O.OracleTextModel(cfg, w).forward_rows([rows[r] for r in pick], threads=16)
    worst_abs, worst_cos = 0.0, 1.0
    for r, o in zip(pick, ref):
        off = 0
        for d in DIMS:
            want = O.truncate_and_normalize(o["normalized"], d)
            have = got[r, off:off + d]
            a = float(np.abs(have - want).max())
            c = cosine(have, want)
            worst_abs, worst_cos = max(worst_abs, a), min(worst_cos, c)
            assert a <= MAX_ABS and c >= MIN_COS, \
                f"row {r} (len {lengths[r]}) dim {d}: max-abs {a:.3g} cosine {c:.8f}"
            off += d
    print(f"headline batch: {len(pick)} rows x {len(DIMS)} dims, worst max-abs {worst_abs:.3g}, "
          f"worst cosine {worst_cos:.8f}", flush=True)


@pytest.mark.gpu
def test_shape_b_headline_batch_matches_oracle():
    """The same 64-row batch through the reference manifest's shape (hidden
    512, 4 query heads, 2 KV heads of 256 on sliding layers and 1 KV head of
    512 on the 4 global layers, FFN 2048, PLE 512) at 24 layers and vocab
    262144, three row groups; 8 rows (two per quarter of the batch) against
    the oracle at every Matryoshka dim."""
    cfg = svl_synth.config_b()
    w = svl_synth.weights(cfg, seed=0)
    lengths = svl_synth.row_lengths(BATCH, LEN_LO, LEN_HI, seed=1)
    rows = svl_synth.token_rows(cfg["vocab_size"], lengths, seed=1)
    offsets = np.zeros(BATCH + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    m = S.TextModel(S.TextConfig.from_json_value(cfg), w)
    m.set_stream_split(GROUPS)
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    out = torch.zeros((BATCH, sum(DIMS)), dtype=torch.float32, device="cuda:0")
    m.forward_device(ids.data_ptr(), offsets, DIMS, out.data_ptr(),
                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    m.close()
    pick = [int(r) for q in range(4) for r in
            np.random.default_rng(13 + q).choice(np.arange(16 * q, 16 * q + 16), 2, replace=False)]
    ref = O.OracleTextModel(cfg, w).forward_rows([rows[r] for r in pick], threads=8)
    for r, o in zip(pick, ref):
        off = 0
        for d in DIMS:
            want = O.truncate_and_normalize(o["normalized"], d)
            have = got[r, off:off + d]
            a = float(np.abs(have - want).max())
            c = cosine(have, want)
            assert a <= MAX_ABS and c >= MIN_COS, \
                f"row {r} (len {lengths[r]}) dim {d}: max-abs {a:.3g} cosine {c:.8f}"
            off += d
    print(f"shape B batch: rows {pick} match the oracle at dims {DIMS}", flush=True)
