"""Throughput benchmark of the MI355X text encoder.

Workload (one "step" = one forward pass of one batch): the EmbeddingGemma-
shaped FP32 text encoder (hidden 768, 24 layers, 3 query heads sharing one
KV head of dim 256, GeGLU FFN 1152, PLE 256, vocab 262144) with random-init
weights (seed 0), batch 64 rows, row lengths uniform in [64, 512] (seed 1),
token ids uniform over the vocabulary (seed 1), padding masked by packing
the rows back to back, outputs at Matryoshka dims 768 / 512 / 256 / 128.
Token ids are resident in HBM before the timed region; every step runs the
whole encoder and writes the normalised embeddings to HBM.

Prints one JSON line: embeddings/s (value, timed on the production path:
three row groups on three streams), the roofline of the dominant kernel (the
gate/up GEMM; its launches timed with HIP events on the stream they run on,
in a second pass of the same steps on one stream so that each kernel's
duration is its own), the CPU oracle timed on this host's cores on a bounded
sample of the batch's rows, and the parity of those rows of the timed output
against the oracle's. Secondary legs, each with its own workload string: the
same batch from host ids to host vectors, 8 x 2048-token rows, image prompts
(vision tower + text encoder), audio prompts (audio tower + text encoder,
from log-mel frames and from 16 kHz samples through the log-mel front end),
and exact cosine search over a 1M x 768 index.
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "seldon-vault-lite-rust_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "text embeddings/sec at batch 64×seq 512 FP32; % FP32-MFMA peak; p50 latency"
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X published dense FP32 matrix peak
PEAK_HBM_GBS = 8000.0
PEAK_FP64_TFLOPS = 78.6  # MI355X published FP64 peak
BATCH, LEN_LO, LEN_HI = 64, 64, 512
DIMS = [768, 512, 256, 128]


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--cpu-sample-rows", type=int, default=-1,
                    help="rows of the workload timed on the CPU oracle (default: two per worker "
                         "thread, at most 16 threads; 0 skips the CPU baseline)")
    ap.add_argument("--t1-runs", type=int, default=20)
    ap.add_argument("--image-steps", type=int, default=5,
                    help="timed batches of the image workload (0 skips it)")
    ap.add_argument("--audio-steps", type=int, default=5,
                    help="timed batches of the audio workload (0 skips it)")
    ap.add_argument("--search-steps", type=int, default=5,
                    help="timed batches of the vector-search workload (0 skips it)")
    ap.add_argument("--long-steps", type=int, default=5,
                    help="timed batches of the 8 x 2048-token workload (0 skips it)")
    ap.add_argument("--shape-b-steps", type=int, default=10,
                    help="timed batches of the headline batch at the manifest shape (0 skips it)")
    ap.add_argument("--host-steps", type=int, default=10,
                    help="timed batches of the host-ids to host-vectors path (0 skips it)")
    ap.add_argument("--row-groups", type=int, default=3,
                    help="row groups (streams) the batch is split into")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device-to-device copy (3 times), the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings")
    return ap.parse_args()


def copy_calibration():
    import torch

    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "bytes_written": n * 4,
                      "launches": 3}), flush=True)


def gemm_traffic():
    """HBM bytes per launch of the gate/up GEMM from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor),
    or None when no such measurement is committed."""
    path = os.path.join(ROOT, "profiles", "gemm_gate_up_T2_hbm_traffic.md")
    if not os.path.exists(path):
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read())
    return float(m.group(1)) if m else None


def host_cpu():
    """nproc (logical CPUs of the host), the CPUs this process may run on, and
    the CPU model string from /proc/cpuinfo."""
    model = None
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return os.cpu_count(), usable, model


def cpu_baseline(cfg, weights, rows_all, n_rows, gpu_out):
    """The scalar C oracle (the reference's x86-64 path restated) on a seeded
    subset of the batch's rows, pulled by worker threads from one queue as
    the reference's request-level bench does (tests/text_bench.rs:58-72), on
    at most 16 threads: the host share of one GPU on the MI355X boxes. The
    same rows of the GPU output are compared with the oracle's, giving the
    line's parity object."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    from oracle import oracle as O

    if n_rows == 0:
        return None, None
    nproc, usable, model_name = host_cpu()
    threads = max(1, min(usable, 16))
    n = n_rows if n_rows > 0 else 2 * threads
    pick = sorted(int(i) for i in np.random.default_rng(12).choice(len(rows_all), n, replace=False))
    rows = [rows_all[i] for i in pick]
    oracle = O.OracleTextModel(cfg, weights)
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        outs = list(ex.map(lambda r: oracle.forward(r), rows))
    wall = time.perf_counter() - t0
    toks = sum(len(r) for r in rows)
    cpu = {"value": n / wall, "unit": "embeddings/s", "cores": threads, "kind": "port",
           "nproc": nproc, "usable_cpus": usable, "cpu_model": model_name,
           "sample": f"{n} rows of the same batch (seeded subset, {toks} tokens, lengths "
                     f"{min(len(r) for r in rows)}-{max(len(r) for r in rows)}), pulled from one "
                     f"queue by {threads} worker threads, scalar C oracle (-O2, no FMA "
                     f"contraction), {wall:.1f} s wall"}
    worst_abs, worst_cos = 0.0, 1.0
    for i, o in zip(pick, outs):
        off = 0
        for d in DIMS:
            want = O.truncate_and_normalize(o["normalized"], d).astype(np.float64)
            have = gpu_out[i, off:off + d].astype(np.float64)
            worst_abs = max(worst_abs, float(np.abs(have - want).max()))
            worst_cos = min(worst_cos, float(have @ want / (np.linalg.norm(have)
                                                             * np.linalg.norm(want))))
            off += d
    parity = {"rows": n, "dims": DIMS, "max_abs": worst_abs, "min_cos": worst_cos,
              "tolerance": {"max_abs": 1e-4, "min_cos": 0.99999},
              "ok": bool(worst_abs <= 1e-4 and worst_cos >= 0.99999),
              "against": "scalar C oracle, same rows of the timed batch's output"}
    return cpu, parity


def shape_b_leg(rows, offsets, steps, groups):
    """The headline batch (same 64 rows and ids) through the reference
    manifest's own shape: hidden 512, 4 query heads, 2 KV heads of 256 on the
    20 sliding layers and 1 KV head of 512 on the 4 global layers, FFN 2048,
    PLE 512, vocab 262144, random-init weights (seed 0)."""
    import numpy as np
    import torch

    import svl_amd
    import svl_synth

    cfg = svl_synth.config_b()
    w = svl_synth.weights(cfg, seed=0)
    model = svl_amd.TextModel(svl_amd.TextConfig.from_json_value(cfg), w)
    del w
    model.set_stream_split(groups)
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    out = torch.zeros((len(rows), sum(DIMS)), dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        model.forward_device(ids.data_ptr(), offsets, DIMS, out.data_ptr(), stream)

    step()
    torch.cuda.synchronize()
    ms = []
    for _ in range(steps):
        a = time.perf_counter()
        step()
        torch.cuda.synchronize()
        ms.append((time.perf_counter() - a) * 1e3)
    p50 = float(np.median(ms))
    assert np.isfinite(out.cpu().numpy()).all()
    # kernel pass: one untimed single-stream step first (the workspace of the
    # single-group layout), then one step with HIP events around every launch
    model.set_stream_split(False)
    step()
    torch.cuda.synchronize()
    model.set_kernel_timing(True)
    step()
    torch.cuda.synchronize()
    stats = model.kernel_stats()
    model.close()
    attn = stats["attention"]
    gemm_keys = [k for k in stats if k.startswith("gemm_")]
    gemm_ms = sum(stats[k]["ms"] for k in gemm_keys)
    gemm_flops = sum(stats[k]["work"] for k in gemm_keys)
    flops = gemm_flops + attn["work"]
    return {"workload": "the headline batch (64 rows, lengths U[64,512], seed 1) through the "
                        "reference manifest's shape: hidden 512, 4 q heads, 2 KV heads of 256 on "
                        "20 sliding layers, 1 KV head of 512 on 4 global layers, FFN 2048, PLE "
                        "512, vocab 262144",
            "embeddings_per_s": round(len(rows) / (p50 * 1e-3), 2), "p50_ms": round(p50, 3),
            "forward_tflops": round(flops / (p50 * 1e-3) / 1e12, 2),
            "forward_frac_of_fp32_mfma_peak": round(flops / (p50 * 1e-3) / 1e12
                                                    / PEAK_FP32_MFMA_TFLOPS, 4),
            "gemm_tflops": round(gemm_flops / (gemm_ms * 1e-3) / 1e12, 2),
            "attention_ms_per_batch": round(attn["ms"], 3),
            "attention_tflops": round(attn["work"] / (attn["ms"] * 1e-3) / 1e12, 2),
            "kernels": {k: round(v["ms"], 3) for k, v in stats.items() if v["launches"]},
            "steps": steps}


def long_context_leg(model, steps):
    """Long-context workload: the same text encoder on a batch of 8 rows of
    2048 tokens (ids uniform over the vocabulary, seed 4): 20 sliding-window
    layers (|i - j| <= 512) and 4 global layers. Attention FLOPs are counted
    algorithmically, keys per query inside the window only."""
    import numpy as np
    import torch

    import svl_synth

    n, L = 8, 2048
    rows = svl_synth.token_rows(model.config.vocab_size, [L] * n, seed=4)
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    offsets = np.arange(n + 1, dtype=np.int64) * L
    out = torch.zeros((n, 768), dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream

    def step():
        model.forward_device(ids.data_ptr(), offsets, [768], out.data_ptr(), stream)

    step()
    torch.cuda.synchronize()
    ms = []
    for _ in range(steps):
        a = time.perf_counter()
        step()
        torch.cuda.synchronize()
        ms.append((time.perf_counter() - a) * 1e3)
    p50 = float(np.median(ms))
    assert np.isfinite(out.cpu().numpy()).all()
    groups = model.row_groups
    model.set_stream_split(False)
    model.set_kernel_timing(True)
    step()
    torch.cuda.synchronize()
    stats = model.kernel_stats()
    model.set_kernel_timing(False)
    model.set_stream_split(groups)
    attn = stats["attention"]
    gemm_keys = [k for k in stats if k.startswith("gemm_")]
    gemm_ms = sum(stats[k]["ms"] for k in gemm_keys)
    gemm_flops = sum(stats[k]["work"] for k in gemm_keys)
    flops = gemm_flops + attn["work"]
    return {"workload": "the same text encoder on 8 rows x 2048 tokens (ids uniform over the "
                        "vocabulary, seed 4): 20 sliding-window layers (window 512), 4 global",
            "embeddings_per_s": round(n / (p50 * 1e-3), 2), "p50_ms_per_batch": round(p50, 3),
            "forward_tflops": round(flops / (p50 * 1e-3) / 1e12, 2),
            "forward_frac_of_fp32_mfma_peak": round(flops / (p50 * 1e-3) / 1e12
                                                    / PEAK_FP32_MFMA_TFLOPS, 4),
            "attention_flops_per_batch": attn["work"],
            "attention_ms_per_batch": round(attn["ms"], 3),
            "attention_tflops": round(attn["work"] / (attn["ms"] * 1e-3) / 1e12, 2),
            "gemm_tflops": round(gemm_flops / (gemm_ms * 1e-3) / 1e12, 2),
            "kernel_timing": "one pass on one stream, HIP events per launch", "steps": steps}


def image_leg(text_model, dev, steps):
    """Image workload: batch 4 synthetic 768x768 RGB noise images (seed 2),
    48x48 = 2304 patches each, through the 16-layer vision tower (config V,
    random-init weights seed 0) and the text encoder (prompt of 260 tokens
    with the 256 soft tokens substituted). Patches resident in HBM."""
    import numpy as np
    import torch

    import svl_synth
    import svl_vision

    n_img, grid = 4, 48
    c = svl_synth.config_v(16)
    vw = svl_synth.vision_weights(c, 768, seed=0)
    vm = svl_vision.VisionModel(svl_vision.VisionConfig.from_json_value(c), vw, 768, dev)
    del vw
    patches = svl_synth.image_patches(n_img, grid, grid, seed=2)
    src = torch.from_numpy(np.concatenate([p.pixel_values[: p.valid_patches]
                                           for p in patches])).to("cuda:0")
    pix = torch.empty_like(src)
    soft = torch.empty((sum(p.soft_tokens for p in patches), 768), device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    emb = svl_vision.ImageEmbedder(text_model, vm, svl_vision.ImageSpecialTokens())

    def tower():
        pix.copy_(src)  # the tower rescales its input in place
        vm.forward_device(pix.data_ptr(), patches, soft.data_ptr(), stream)

    def embed():
        pix.copy_(src)
        return emb.embed_device(pix.data_ptr(), patches, 768)

    def timed(f):
        f()
        torch.cuda.synchronize()
        ms = []
        for _ in range(steps):
            a = time.perf_counter()
            f()
            torch.cuda.synchronize()
            ms.append((time.perf_counter() - a) * 1e3)
        return float(np.median(ms))

    tower_ms = timed(tower)
    embed_ms = timed(embed)
    out = embed()
    assert np.isfinite(out).all()
    P, H, I, L, hd, nh = grid * grid, 768, 3072, 16, 64, 12
    per_img = (2 * P * 768 * H + L * (2 * P * H * (3 * nh * hd + H + 3 * I) + 4 * hd * nh * P * P)
               + 2 * (P // 9) * H * 768)
    flops = n_img * per_img
    return {"workload": "batch 4 synthetic 768x768 RGB noise images (seed 2), 2304 patches "
                        "each: 16-layer vision tower (hidden 768, 12 heads of 64, FFN 3072) "
                        "+ text encoder over the 260-token image prompt; patches in HBM",
            "images_per_s": round(n_img / (embed_ms * 1e-3), 2),
            "p50_ms_per_batch": round(embed_ms, 3),
            "tower_p50_ms_per_batch": round(tower_ms, 3),
            "tower_tflops": round(flops / (tower_ms * 1e-3) / 1e12, 2),
            "tower_frac_of_fp32_mfma_peak": round(flops / (tower_ms * 1e-3) / 1e12
                                                  / PEAK_FP32_MFMA_TFLOPS, 4),
            "tower_flops_per_batch": flops, "steps": steps}


def audio_leg(text_model, dev, steps, cpu_sample=True):
    """Audio workload: batch 4 clips of 30 s of 16 kHz mono audio (three
    sines uniform in 100-4000 Hz plus N(0, 0.05^2) noise, seed 3) resident in
    HBM -> log-mel front end (2999 frames of 128 bins per clip, all valid) ->
    12-layer audio tower (config AU, random-init weights seed 0; 750 audio
    tokens per clip) -> text encoder over the 754-token audio prompt ->
    768-d embeddings. Each stage is also timed alone on the same data."""
    import numpy as np
    import torch

    import svl_audio
    import svl_synth

    n_clip, frames = 4, 2999
    c = svl_synth.config_au(12)
    aw = svl_synth.audio_weights(c, 768, seed=0)
    am = svl_audio.AudioModel(svl_audio.AudioConfig.from_json_value(c), aw, 768, dev)
    del aw
    clips = svl_synth.sine_clips(n_clip, seed=3)
    lengths = [x.size for x in clips]
    samples = torch.from_numpy(np.concatenate(clips)).to("cuda:0")
    feats = torch.empty((n_clip * frames, 128), device="cuda:0")
    lm = svl_audio.LogMel(dev)
    masks = lm.compute_device(samples.data_ptr(), lengths, feats.data_ptr())
    torch.cuda.synchronize()
    host_feats = feats.cpu().numpy()
    mels = [svl_audio.MelSpectrogram(host_feats[i * frames:(i + 1) * frames], masks[i])
            for i in range(n_clip)]
    assert all(m.frames == frames and m.valid_frames() == frames for m in mels)
    tokens = sum(m.audio_tokens() for m in mels)
    soft = torch.empty((tokens, 768), device="cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    emb = svl_audio.AudioEmbedder(text_model, am, svl_audio.AudioSpecialTokens())

    def timed(f):
        f()
        torch.cuda.synchronize()
        ms = []
        for _ in range(steps):
            a = time.perf_counter()
            f()
            torch.cuda.synchronize()
            ms.append((time.perf_counter() - a) * 1e3)
        return float(np.median(ms))

    mel_ms = timed(lambda: lm.compute_device(samples.data_ptr(), lengths, feats.data_ptr()))
    tower_ms = timed(lambda: am.forward_device(feats.data_ptr(), mels, soft.data_ptr(), stream))
    embed_ms = timed(lambda: emb.embed_device(feats.data_ptr(), mels, 768))
    samples_ms = timed(lambda: emb.embed_samples_device(samples.data_ptr(), lengths, 768))
    out = emb.embed_samples_device(samples.data_ptr(), lengths, 768)
    assert np.isfinite(out).all()
    cpu_mel = None
    if cpu_sample:
        from oracle import oracle as O
        a = time.perf_counter()
        O.log_mel(clips[0])
        cpu_mel_s = time.perf_counter() - a
        cpu_mel = {"value": round(1.0 / cpu_mel_s, 3), "unit": "clips/s", "cores": 1,
                   "kind": "port", "sample": "one 30 s clip through the C oracle log_mel"}
    H, L, C0, C1, P, T = 1024, 12, 128, 32, 1536, tokens // n_clip
    f1 = (frames + 1) // 2
    per_clip = (2 * f1 * 64 * C0 * 9 + 2 * T * 32 * C1 * C0 * 9 + 2 * T * 32 * C1 * H
                + L * 2 * T * H * (2 * 2 * 4 * H + 3 * H + H + 2 * H + H)
                + L * 4 * 8 * 128 * T * 12 + 2 * T * H * P + 2 * T * P * 768)
    flops = n_clip * per_clip
    return {"workload": "batch 4 clips of 30 s of 16 kHz mono audio in HBM (3 sines uniform in "
                        "100-4000 Hz + N(0, 0.05^2) noise, seed 3) -> log-mel (2999 frames x 128) "
                        "-> 12-layer audio tower (hidden 1024, 8 heads of 128, SSCP [128, 32], "
                        "chunk 12; 750 tokens per clip) -> text encoder over the 754-token "
                        "audio prompt",
            "clips_per_s": round(n_clip / (samples_ms * 1e-3), 2),
            "p50_ms_per_batch": round(samples_ms, 3),
            "tower_p50_ms_per_batch": round(tower_ms, 3),
            "tower_tflops": round(flops / (tower_ms * 1e-3) / 1e12, 2),
            "tower_frac_of_fp32_mfma_peak": round(flops / (tower_ms * 1e-3) / 1e12
                                                  / PEAK_FP32_MFMA_TFLOPS, 4),
            "tower_flops_per_batch": flops, "steps": steps,
            "log_mel": {"workload": "the same 4 clips: samples in HBM -> [4 x 2999, 128] "
                                    "log-mel features in HBM (f64 FFT, bit-exact with the "
                                    "reference)",
                        "clips_per_s": round(n_clip / (mel_ms * 1e-3), 2),
                        "p50_ms_per_batch": round(mel_ms, 3),
                        "frames_per_s": round(n_clip * frames / (mel_ms * 1e-3), 1),
                        "cpu_baseline": cpu_mel},
            "from_log_mel": {"clips_per_s": round(n_clip / (embed_ms * 1e-3), 2),
                             "p50_ms_per_batch": round(embed_ms, 3)}}


def search_leg(dev, steps, cpu_sample=True):
    """Exact cosine search: an index of 1,000,000 chunk embeddings of
    dimension 768 (U(-1, 1), seed 5; chunk ids 1..n) resident in HBM; a batch
    of 64 queries (seed 6) ranked in full and sliced to the top 10, and one
    query alone. Scores are the reference's f64 sequential dot products; the
    work is 2 * n * 768 FLOP (f64 FMA) per query."""
    import numpy as np
    import torch

    import svl_amd
    import svl_search

    n, d, nq, k = 1_000_000, 768, 64, 10
    emb = svl_amd.synth_uniform(5, 0, -1.0, 1.0, n * d).reshape(n, d)
    ids = np.arange(1, n + 1, dtype=np.uint64)
    ix = svl_search.VectorIndex(emb, ids, dev)
    qs = svl_amd.synth_uniform(6, 0, -1.0, 1.0, nq * d).reshape(nq, d)
    dq = torch.from_numpy(qs).to("cuda:0")
    torch.cuda.synchronize()

    def timed(f, reps):
        f()
        ms = []
        for _ in range(reps):
            a = time.perf_counter()
            f()
            ms.append((time.perf_counter() - a) * 1e3)
        return float(np.median(ms))

    batch_ms = timed(lambda: ix.rank_device(dq.data_ptr(), nq, d, limit=k), steps)
    one_ms = timed(lambda: ix.rank_device(dq.data_ptr(), 1, d, limit=k), steps)
    flops = 2.0 * n * d * nq
    # the FP64 matrix rate this device sustains on register-only MFMA chains
    fp64_peak = dev.measure_fp64_peak()
    cpu = None
    if cpu_sample:
        from oracle import oracle as O
        a = time.perf_counter()
        O.vector_rank(qs[0], emb, ids)
        cpu_s = time.perf_counter() - a
        cpu = {"value": round(1.0 / cpu_s, 3), "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": "one query over the full 1M x 768 index through the C oracle "
                         "vector_rank (f64 sequential dot products and the full sort)"}
    del emb
    return {"workload": "exact cosine ranking, 1,000,000 x 768 f32 chunk embeddings in HBM, "
                        "64 queries in HBM, full ranking per query sliced to the top 10",
            "queries_per_s": round(nq / (batch_ms * 1e-3), 1),
            "p50_ms_per_batch": round(batch_ms, 3),
            "one_query_p50_ms": round(one_ms, 3),
            "f64_tflops_wall": round(flops / (batch_ms * 1e-3) / 1e12, 2),
            "frac_of_fp64_peak_wall": round(flops / (batch_ms * 1e-3) / 1e12 / PEAK_FP64_TFLOPS, 4),
            "measured_fp64_mfma_tflops": round(fp64_peak, 2),
            "frac_of_measured_fp64_wall": round(flops / (batch_ms * 1e-3) / 1e12 / fp64_peak, 4),
            "cpu_baseline": cpu, "steps": steps}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: the benchmark runs on one GPU; --gpus {args.gpus} is not supported "
              f"(rows are independent and would shard by data parallelism)",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration()
        return

    import numpy as np
    import torch

    import svl_amd
    import svl_synth

    torch.cuda.set_device(0)
    dev = svl_amd.Device.get(0)
    mfma_peak, hbm_peak = dev.measure_peaks()
    cfg = svl_synth.config_a()
    weights = svl_synth.weights(cfg, seed=0)
    lengths = svl_synth.row_lengths(BATCH, LEN_LO, LEN_HI, seed=1)
    rows = svl_synth.token_rows(cfg["vocab_size"], lengths, seed=1)
    model = svl_amd.TextModel(svl_amd.TextConfig.from_json_value(cfg), weights, dev)

    offsets = np.zeros(BATCH + 1, np.int64)
    offsets[1:] = np.cumsum(lengths)
    T = int(offsets[-1])
    ids = torch.from_numpy(np.concatenate(rows).astype(np.int32)).to("cuda:0")
    out = torch.zeros((BATCH, sum(DIMS)), dtype=torch.float32, device="cuda:0")
    stream = torch.cuda.current_stream()

    model.set_stream_split(args.row_groups)

    def step():
        model.forward_device(ids.data_ptr(), offsets, DIMS, out.data_ptr(), stream.cuda_stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region: K steps of the production path (row groups on their own
    # streams, three by default), bracketed by device synchronisation.
    step_ms = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        a = time.perf_counter()
        step()
        step_ms.append((time.perf_counter() - a) * 1e3)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # Kernel pass: the same K steps on one stream, with HIP events recorded
    # around every launch on the stream it runs on, so each kernel's duration
    # is its own (not shared with the other row group's kernels).
    model.set_stream_split(False)
    model.set_kernel_timing(True)
    torch.cuda.synchronize()
    k0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    single_stream_ms = (time.perf_counter() - k0) * 1e3 / args.steps
    stats = model.kernel_stats()
    model.set_kernel_timing(False)
    model.set_stream_split(args.row_groups)

    value = BATCH * args.steps / elapsed
    ms_per_step = elapsed * 1e3 / args.steps
    p50 = float(np.median(step_ms))

    # Dominant kernel: the fused gate/up GEMM with GeGLU epilogue.
    gu = stats["gemm_gate_up"]
    gu_ms = gu["ms"] / max(gu["launches"], 1)
    gu_flops = gu["work"] / max(gu["launches"], 1)
    gu_tflops = gu_flops / (gu_ms * 1e-3) / 1e12
    gemm_keys = [k for k in stats if k.startswith("gemm_")]
    gemm_ms = sum(stats[k]["ms"] for k in gemm_keys)
    gemm_flops = sum(stats[k]["work"] for k in gemm_keys)
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0
    attn = stats["attention"]
    attn_tflops = attn["work"] / (attn["ms"] * 1e-3) / 1e12 if attn["ms"] else 0.0
    fwd_flops = (gemm_flops + attn["work"]) / args.steps
    total_kernel_ms = sum(v["ms"] for v in stats.values()) / args.steps

    # The timed batch's output, for the parity check against the oracle.
    step()
    torch.cuda.synchronize()
    gpu_out = out.cpu().numpy()

    # The same batch from ids on the host to Matryoshka vectors on the host
    # (PCIe upload of the ids and download of the embeddings included), two
    # ways: the serving path (pinned host buffers, forward_device), and the
    # host-buffer API (svl_text_forward_batch, then truncate_and_normalize per
    # row and dimension through the C ABI from Python).
    host = None
    if args.host_steps > 0:
        ids_host = torch.empty(ids.shape, dtype=ids.dtype, pin_memory=True)
        ids_host.copy_(torch.from_numpy(np.concatenate(rows).astype(np.int32)))
        out_host = torch.empty(out.shape, dtype=out.dtype, pin_memory=True)
        ids_dev = torch.empty_like(ids)

        def host_step():
            ids_dev.copy_(ids_host, non_blocking=True)
            model.forward_device(ids_dev.data_ptr(), offsets, DIMS, out.data_ptr(),
                                 stream.cuda_stream)
            out_host.copy_(out, non_blocking=True)
            stream.synchronize()

        host_step()
        sms = []
        for _ in range(args.host_steps):
            a = time.perf_counter()
            host_step()
            sms.append((time.perf_counter() - a) * 1e3)
        assert np.array_equal(out_host.numpy(), gpu_out)
        model.embed_batch(rows, DIMS)
        hms = []
        for _ in range(args.host_steps):
            a = time.perf_counter()
            hv = model.embed_batch(rows, DIMS)
            hms.append((time.perf_counter() - a) * 1e3)
        # the host truncation sums in order, the device's in a tree: last-bit
        # differences only
        assert np.abs(hv - gpu_out).max() <= 1e-6
        sp50, hp50 = float(np.median(sms)), float(np.median(hms))
        host = {"embeddings_per_s": round(BATCH / (sp50 * 1e-3), 3), "p50_ms": round(sp50, 3),
                "span": "token ids in pinned host memory -> upload -> forward_device with the "
                        "Matryoshka dims -> 64 x (768/512/256/128) vectors downloaded to pinned "
                        "host memory",
                "host_buffer_api": {
                    "embeddings_per_s": round(BATCH / (hp50 * 1e-3), 3), "p50_ms": round(hp50, 3),
                    "span": "token ids in host memory -> svl_text_forward_batch -> normalized "
                            "vectors in host memory -> svl_truncate_and_normalize per row and "
                            "dimension (256 calls from Python)"},
                "steps": args.host_steps}

    # Single-request latency: batch 1 x 128 tokens.
    t1_ids = torch.from_numpy(svl_synth.token_rows(cfg["vocab_size"], [128], seed=1)[0]
                              .astype(np.int32)).to("cuda:0")
    t1_off = np.array([0, 128], np.int64)
    t1_out = torch.zeros((1, 768), dtype=torch.float32, device="cuda:0")
    lat = []
    for i in range(args.t1_runs + 2 if args.t1_runs > 0 else 0):
        a = time.perf_counter()
        model.forward_device(t1_ids.data_ptr(), t1_off, [768], t1_out.data_ptr(), stream.cuda_stream)
        if i >= 2:
            lat.append((time.perf_counter() - a) * 1e3)

    traffic = gemm_traffic()
    roofline = {"kernel": "gemm_nt_dma<64,128,16,EPI_GEGLU,4,2,2> (gate/up projection + GeGLU)",
                "bound": "mfma", "achieved": round(gu_tflops, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(gu_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
                "traffic": traffic,
                "flops_per_launch": gu_flops, "avg_launch_ms": round(gu_ms, 4),
                "launches": gu["launches"]}

    image = image_leg(model, dev, args.image_steps) if args.image_steps > 0 else None
    audio = (audio_leg(model, dev, args.audio_steps, args.cpu_sample_rows != 0)
             if args.audio_steps > 0 else None)
    search = (search_leg(dev, args.search_steps, args.cpu_sample_rows != 0)
              if args.search_steps > 0 else None)
    long_ctx = long_context_leg(model, args.long_steps) if args.long_steps > 0 else None
    shape_b = (shape_b_leg(rows, offsets, args.shape_b_steps, args.row_groups)
               if args.shape_b_steps > 0 else None)
    cpu, parity = cpu_baseline(cfg, weights, rows, args.cpu_sample_rows, gpu_out)

    breakdown = {k: {"ms_per_step": round(v["ms"] / args.steps, 3),
                     "launches_per_step": v["launches"] // max(args.steps, 1)}
                 for k, v in stats.items() if v["launches"]}
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "embeddings/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random-init weights seed 0, token ids and row lengths seed 1)",
        "config": {"workload": "EmbeddingGemma-shaped FP32 text encoder forward (hidden 768, 24 "
                               "layers, 3 q heads / 1 KV head, head_dim 256, GeGLU 1152, PLE 256, "
                               "vocab 262144): batch 64 rows, lengths U[64,512], padding masked, "
                               "Matryoshka outputs 768/512/256/128",
                   "batch": BATCH, "tokens": T, "max_seq_len": LEN_HI, "parallelism": "single GPU",
                   "row_groups": args.row_groups},
        "p50_ms": round(p50, 3),
        "t1_p50_ms": round(float(np.median(lat)), 3) if lat else None,
        "gemm_tflops": round(gemm_tflops, 3),
        "gemm_frac_of_fp32_mfma_peak": round(gemm_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
        "attention_tflops": round(attn_tflops, 3),
        "forward_tflops": round(fwd_flops / (ms_per_step * 1e-3) / 1e12, 3),
        "forward_frac_of_fp32_mfma_peak": round(fwd_flops / (ms_per_step * 1e-3) / 1e12
                                                / PEAK_FP32_MFMA_TFLOPS, 4),
        "kernel_ms_per_step": round(total_kernel_ms, 3),
        "single_stream_ms_per_step": round(single_stream_ms, 3),
        "roofline": roofline,
        "measured_peaks": {"fp32_mfma_tflops": round(mfma_peak, 2),
                           "hbm_copy_gbs": round(hbm_peak, 1),
                           "method": "register-only MFMA chains on every SIMD (16 chains of "
                                     "16x16x4 f32 in one wave per SIMD, 4 chains of 32x32x2 f32 "
                                     "in two; the faster); 1 GiB device-to-device copy, one "
                                     "float4 per thread (read + written bytes); best of a few "
                                     "launches each",
                           "published": {"fp32_mfma_tflops": PEAK_FP32_MFMA_TFLOPS,
                                         "hbm_gbs": PEAK_HBM_GBS}},
        "cpu_baseline": cpu,
        "parity": parity,
        "host_to_host": host,
        "kernels": breakdown,
        "long_context": long_ctx,
        "shape_b": shape_b,
        "image": image,
        "audio": audio,
        "search": search,
    }
    if cpu:
        line["speedup_vs_cpu_baseline"] = round(value / cpu["value"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
