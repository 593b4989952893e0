"""Decode benchmark: Llama-3-8B-shape Q4_0 greedy decode on one MI355X.

Workload (headline metric "decode tok/s, Llama-3-8B-shape Q4_0, bs=1 &
32; GEMV HBM GB/s vs peak"):
  * value: batch-1 greedy decode tok/s of a random-init Llama-3-8B-architecture
    model (32 layers, hidden 4096, 32/8 heads, FFN 14336, vocab 128256, RoPE
    theta 5e5) with Q4_0 block weights, an F16 LM head, an fp16 KV cache and
    fp16 activations into the products, created at Llama-3-8B's 8192-token
    context. A 128-token prompt is prefilled, then each timed step is one
    HIP-graph decode step (embed -> 32 layers -> LM head -> argmax fed back as
    the next token).
  * bs32: the ragged continuous-batch step of benchmark configuration 5 (32 sequences,
    fp16 KV contexts uniform in [256, 4096], one forward pass per step).
  * roofline: the dominant kernel, the Q4_0 GEMV at the 14336x4096 decode shape
    (config 2: x fp16, fp32 accumulate, fp16 output), timed with HIP events over
    graph-replayed back-to-back launches rotating through > 256 MB of weight
    copies so the Infinity Cache cannot serve them.
  * gemm_m32_q4_0: the config-5 small-M product at the four layer shapes
    (32 binary16 rows, MFMA GEMM + split-K reduce), GB/s and the fraction of
    dense fp16 MFMA peak.
  * llama2_7b_q4k_c3: config 3 (Llama-2-7B shape, Q4_K, decode to 2048 ctx).
  * attention_c4: config 4 (16 ragged sequences, GQA 32/8, fp16 KV).
  * bs1_penalty / bs1_reference_dtype: the same batch-1 decode with the
    reference's default greedy sampler in the captured step (repetition
    penalty 1.15 over the generated tokens, last-max argmax), and with the
    reference's dtypes (f32 activations into the products, f32 KV).
  * in_step: per-kernel HBM fractions inside the batch-1 decode step, from the
    kernel trace committed in profiles/ (bytes computed here from the shapes).
  * cpu_baseline: the CPU oracle (a restatement of the reference arithmetic, not
    the reference itself) on the same model, OpenMP over rows on every host
    core, median per-token time of a bounded sample.

Every timed leg reports the median of its trials.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0    # dense fp16 MFMA, MI355X
PROFILES = ROOT / "profiles"
METRIC = "decode tok/s, Llama-3-8B-shape Q4_0, bs=1 & 32; GEMV HBM GB/s vs peak"
L3 = dict(hidden=4096, heads=32, kv_heads=8, ffn=14336, vocab=128256, layers=32, rope_theta=500000.0)
# Llama-3-8B's context: batch-1 models are created with it, so the captured
# step runs the attention plan for the live context length (the length
# bucket that covers it), as for a model loaded at its full context.
L3_CTX = 8192


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def profile_record(name: str) -> dict | None:
    """The machine-readable block (a ```json fence) of profiles/<name>.md: the
    figures a rocprofv3 run gave, with the commit it ran at."""
    path = PROFILES / f"{name}.md"
    if not path.exists():
        return None
    text = path.read_text()
    start = text.find("```json")
    if start < 0:
        return None
    end = text.find("```", start + 7)
    return json.loads(text[start + 7:end])


HEADLINE_TRIALS = 5   # the headline value is the median of this many timed runs of --steps steps


def median_ms(run, trials: int = 5) -> float:
    """Median over `trials` of HIP-event time (ms) around run() on torch's
    current stream (where every timed launch here is enqueued)."""
    import torch
    times = []
    for _ in range(trials):
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        run()
        e.record()
        torch.cuda.synchronize()
        times.append(s.elapsed_time(e))
    return float(np.median(times))


def llama3_spec(seed: int, layers: int = 32):
    from janus_amd import synth
    return synth.make_model(seed, L3["hidden"], L3["heads"], L3["kv_heads"], L3["ffn"], L3["vocab"], layers,
                            synth.Q4_0, 1e-5, L3["rope_theta"], embed_type=synth.F16, head_type=synth.F16)


def decode_bs1(engine, spec, steps: int, warmup: int, prompt_len: int = 128, penalty: float | None = None,
               f32: bool = False, trials: int = 5):
    """Batch-1 greedy decode: prefill token by token, then `steps` captured
    decode steps per trial (the median of `trials` is returned, in ms for the
    `steps` steps). penalty: the reference's default sampler in the captured
    step (repetition penalty over the generated tokens, last-max argmax);
    otherwise plain last-max argmax. f32: the reference's dtypes (f32
    activations into the products, f32 KV)."""
    from janus_amd import _lib
    from janus_amd.model import Model
    max_seq = max(L3_CTX, prompt_len + warmup + trials * steps + 8)
    dt = _lib.DT_F32 if f32 else _lib.DT_F16
    m = Model(engine, spec, max_seq_len=max_seq, kv_dtype=dt, act_dtype=dt)
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, spec.vocab, prompt_len).tolist()
    for p, t in enumerate(prompt):           # prefill token by token (generation.rs:161-173)
        m.forward([t], [p])
    if penalty is not None:
        m.set_sampler(_lib.SAMPLER_PENALTY, penalty)
    m.graph_begin([prompt[-1]], [prompt_len])
    m.graph_run(warmup)
    engine.sync()
    ms = median_ms(lambda: m.graph_run(steps), trials)
    toks = m.graph_tokens(1)
    m.close()
    return ms, toks


def decode_stream(engine, spec, tokens: int = 96, prompt_len: int = 128):
    """Streaming greedy decode (janus_model_generate_stream, the reference's
    generate_with_callback) with the reference's default sampler: the median
    interval between consecutive callbacks, in ms, over `tokens` tokens after
    one untimed call that captures the step."""
    from janus_amd import _lib
    from janus_amd.model import Model
    m = Model(engine, spec, max_seq_len=max(L3_CTX, prompt_len + tokens + 8), kv_dtype=_lib.DT_F16,
              act_dtype=_lib.DT_F16)
    prompt = np.random.default_rng(6).integers(0, spec.vocab, prompt_len).tolist()
    m.generate_with_callback(prompt, 4, lambda t: True)
    stamps = []
    out = m.generate_with_callback(prompt, tokens, lambda t: stamps.append(time.perf_counter()) or True)
    m.close()
    gaps = np.diff(np.asarray(stamps)) * 1e3
    return (float(np.median(gaps)) if gaps.size else float("nan")), len(out)


L2 = dict(hidden=4096, heads=32, kv_heads=32, ffn=11008, vocab=32000, layers=32, rope_theta=10000.0)


def llama2_q4k_spec(seed: int, layers: int = 32):
    """benchmark configuration 3 architecture (Llama-2-7B: 32 layers, hidden 4096, 32 MHA
    heads, FFN 11008, vocab 32000) with Q4_K blocks quantised from N(0, 0.02).
    Quantising 6.7 B weights in numpy takes minutes, so one 4096x4096, one
    11008x4096 and one 4096x11008 matrix are quantised and their bytes reused
    for every layer's q/k/v/o, gate/up and down (each layer is still uploaded
    and streamed from HBM separately); norms and embeddings are per layer."""
    from janus_amd import synth
    rng = np.random.default_rng(seed)
    h, f, v = L2["hidden"], L2["ffn"], L2["vocab"]
    sq = synth.Tensor("", synth.Q4_K, h, h, synth.random_q4_k(rng, h, h))
    gu = synth.Tensor("", synth.Q4_K, f, h, synth.random_q4_k(rng, f, h))
    dn = synth.Tensor("", synth.Q4_K, h, f, synth.random_q4_k(rng, h, f))
    spec = synth.ModelSpec(h, L2["heads"], L2["kv_heads"], f, v, layers, 1e-5, L2["rope_theta"])
    spec.tensors.append(synth.Tensor("token_embd.weight", synth.F16, v, h,
                                     synth.f16_bits(rng.standard_normal((v, h), dtype=np.float32))))
    norm = lambda: 1 + rng.standard_normal(h, dtype=np.float32) * np.float32(0.02)
    for l in range(layers):
        p = f"blk.{l}."
        spec.tensors.append(synth.Tensor(p + "attn_norm.weight", synth.F32, h, 0, norm()))
        for name in ("attn_q", "attn_k", "attn_v", "attn_output"):
            spec.tensors.append(synth.Tensor(p + name + ".weight", synth.Q4_K, h, h, sq.data))
        spec.tensors.append(synth.Tensor(p + "ffn_norm.weight", synth.F32, h, 0, norm()))
        spec.tensors.append(synth.Tensor(p + "ffn_gate.weight", synth.Q4_K, f, h, gu.data))
        spec.tensors.append(synth.Tensor(p + "ffn_up.weight", synth.Q4_K, f, h, gu.data))
        spec.tensors.append(synth.Tensor(p + "ffn_down.weight", synth.Q4_K, h, f, dn.data))
    spec.tensors.append(synth.Tensor("output_norm.weight", synth.F32, h, 0, norm()))
    spec.tensors.append(synth.Tensor("output.weight", synth.F16, v, h,
                                     synth.f16_bits(rng.standard_normal((v, h), dtype=np.float32) * np.float32(0.02))))
    return spec


def decode_c3(engine, spec, prompt_len: int = 512, ctx: int = 2048):
    """benchmark configuration 3 workload: a 512-token random-id prompt prefilled token
    by token, then greedy decode to a 2048-token context (HIP-graph steps), fp16
    KV, batch 1. Returns (decode ms total, decode tokens, prefill s)."""
    import torch
    from janus_amd import _lib
    from janus_amd.model import Model
    m = Model(engine, spec, max_seq_len=ctx, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
    prompt = np.random.default_rng(3).integers(0, spec.vocab, prompt_len).tolist()
    t0 = time.perf_counter()
    for p, t in enumerate(prompt):
        m.forward([t], [p])
    engine.sync()
    prefill_s = time.perf_counter() - t0
    steps = ctx - prompt_len
    m.graph_begin([prompt[-1]], [prompt_len])   # eager step at position n, then the captured step
    engine.sync()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    m.graph_run(steps - 1)
    e.record()
    e.synchronize()
    ms = s.elapsed_time(e)
    m.close()
    return ms, steps - 1, prefill_s


def decode_bs32(engine, spec, steps: int, warmup: int, trials: int = 5):
    """Config 5: 32 sequences over random fp16 caches at contexts U[256, 4096],
    captured ragged steps; median of `trials` timed runs of `steps` steps (ms)."""
    import torch
    from janus_amd import _lib
    from janus_amd.model import Model
    rng = np.random.default_rng(5)
    lens = rng.integers(256, 4097, 32)
    max_seq = int(lens.max()) + warmup + trials * steps + 8
    m = Model(engine, spec, max_seq_len=max_seq, max_batch=32, kv_dtype=_lib.DT_F16, act_dtype=_lib.DT_F16)
    shape = (spec.layers, 32 * max_seq, spec.kv_heads, spec.head_dim)
    g = torch.Generator(device="cuda").manual_seed(5)
    k = torch.randn(shape, device="cuda", dtype=torch.float16, generator=g)
    v = torch.randn(shape, device="cuda", dtype=torch.float16, generator=g)
    m.set_kv_cache(k, v)
    toks = rng.integers(0, spec.vocab, 32).tolist()
    m.graph_begin(toks, lens.tolist())
    m.graph_run(warmup)
    engine.sync()
    ms = median_ms(lambda: m.graph_run(steps), trials)
    m.close()
    del k, v
    return ms, int(lens.sum())


def _weight_bytes(rng, qtype: int, n: int, k: int) -> np.ndarray:
    """GGUF bytes of an [n][k] weight. K-quants quantise 512 N(0, 0.02) rows and
    repeat them (quantising 58 M weights in numpy takes seconds; the bytes
    streamed per launch are the same)."""
    from janus_amd import synth
    if qtype == 2:
        return synth.random_q4_0(rng, n, k)
    rows = min(n, 512)
    gen = {12: synth.random_q4_k, 13: synth.random_q5_k}[qtype]
    base = gen(rng, rows, k).reshape(rows, -1)
    return np.ascontiguousarray(np.tile(base, ((n + rows - 1) // rows, 1))[:n]).reshape(-1)


def gemv_roofline(engine, n: int = 14336, k: int = 4096, launches: int = 200, qtype: int = 2):
    """HIP-event timing of back-to-back GEMV launches (Q4_0 unless qtype says
    otherwise) captured in a graph."""
    import torch
    from janus_amd import ops
    rng = np.random.default_rng(2)
    raw = _weight_bytes(rng, qtype, n, k)
    nbytes = raw.nbytes
    copies = max(2, int(np.ceil(400e6 / nbytes)))
    ws = [ops.GpuTensor(engine, qtype, n, k, raw) for _ in range(copies)]
    x = torch.from_numpy(rng.standard_normal(k).astype(np.float16)).cuda()
    y = torch.empty(n, dtype=torch.float16, device="cuda")
    for i in range(copies):
        ops.gemm_auto(engine, x, ws[i], y, 1, 1, k, n)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        engine.bind_stream(side)
        with torch.cuda.graph(graph, stream=side):
            for i in range(launches):
                ops.gemm_auto(engine, x, ws[i % copies], y, 1, 1, k, n)
    engine.bind_stream()
    graph.replay()
    torch.cuda.synchronize()
    us = median_ms(graph.replay) * 1e3 / launches
    algo = nbytes + 2 * k + 2 * n     # weights once, x in, y out (fp16)
    del graph, ws
    return us, algo, copies


def gemm_m32(engine, n: int, k: int, rows: int = 32, launches: int = 100, qtype: int = 2):
    """The small-M product of config 5 at one layer shape: 32 binary16 rows x a
    quantised weight (Q4_0 unless qtype says otherwise; MFMA GEMM + split-K
    reduce, fp16 output) through janus_gemm_auto, graph-replayed over > 400 MB
    of weight copies. Returns (us per launch, algorithmic bytes, flops)."""
    import torch
    from janus_amd import ops
    rng = np.random.default_rng(12)
    raw = _weight_bytes(rng, qtype, n, k)
    copies = max(2, int(np.ceil(400e6 / raw.nbytes)))
    ws = [ops.GpuTensor(engine, qtype, n, k, raw) for _ in range(copies)]
    a = torch.from_numpy(rng.standard_normal((rows, k)).astype(np.float16)).cuda()
    y = torch.empty(rows, n, dtype=torch.float16, device="cuda")
    for i in range(copies):
        ops.gemm_auto(engine, a, ws[i], y, rows, 1, k, n)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        engine.bind_stream(side)
        with torch.cuda.graph(graph, stream=side):
            for i in range(launches):
                ops.gemm_auto(engine, a, ws[i % copies], y, rows, 1, k, n)
    engine.bind_stream()
    graph.replay()
    torch.cuda.synchronize()
    us = median_ms(graph.replay) * 1e3 / launches
    del graph, ws
    return us, raw.nbytes + 2 * rows * k + 2 * rows * n, 2.0 * rows * n * k


def attention_c4(engine, reps: int = 20):
    """benchmark configuration 4: 16 ragged sequences, ctx ~ U[128, 8192], 32 query / 8 KV
    heads, head_dim 128, fp16 Q/K/V ~ N(0, 1), scale 1/sqrt(128), fp32 softmax,
    packed into one launch through a prefix-sum row-offset table. Returns
    (us per launch, algorithmic bytes, total context)."""
    import torch
    from janus_amd import ops
    rng = np.random.default_rng(4)
    lens = rng.integers(128, 8193, 16)
    base = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int32)
    rows = int(lens.sum())
    g = torch.Generator(device="cuda").manual_seed(4)
    k = torch.randn(rows, 8, 128, device="cuda", generator=g).to(torch.float16)
    v = torch.randn(rows, 8, 128, device="cuda", generator=g).to(torch.float16)
    q = torch.randn(16, 32, 128, device="cuda", generator=g).to(torch.float16).float()
    out = torch.empty(16, 32, 128, device="cuda")
    d_base = torch.from_numpy(base).cuda()
    d_lens = torch.from_numpy(lens.astype(np.int32)).cuda()
    call = lambda: ops.compute_attention(engine, q, k, v, out, 16, 0, rows, 32, 8, 128, row_base=d_base,
                                         seq_lens=d_lens, max_len_hint=int(lens.max()))
    call()
    torch.cuda.synchronize()

    def run():
        for _ in range(reps):
            call()
    us = median_ms(run) * 1e3 / reps
    algo = rows * 8 * 128 * 2 * 2 + q.numel() * 4 + out.numel() * 4
    del k, v
    return us, algo, rows


def copy_bandwidth(nbytes: int = 1 << 30, reps: int = 10):
    """HBM copy rate of torch's device copy over `nbytes` (read + write), the
    practical ceiling a streaming kernel can reach on this box, and the
    calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    ms = median_ms(lambda: dst.copy_(src), reps)
    del src, dst
    return 2 * nbytes / (ms * 1e-3) / 1e9


def cpu_baseline(spec, tokens: int = 20):
    """The oracle (CPU restatement of the reference path, products OpenMP over
    rows on every host core) on a bounded sample: `tokens` greedy decode
    tokens at positions 0.. of the same model, each timed alone; returns
    (tok/s from the median token time, threads, total seconds)."""
    from oracle import oracle as O
    m = O.OracleModel(spec, max_seq_len=tokens + 1, kv_f16=True)
    times = []
    tok = 1
    for p in range(tokens):
        t0 = time.perf_counter()
        logits = m.forward(tok, p)
        tok = O.argmax_last(logits)
        times.append(time.perf_counter() - t0)
    return 1.0 / float(np.median(times)), int(O.lib().jo_num_threads()), float(sum(times))


def in_step_fractions(prompt_len: int = 128) -> dict | None:
    """Per-kernel HBM fractions of the batch-1 decode step from the committed
    kernel trace (profiles/decode_bs1_llama3_8b_q4_0.md): average launch time
    of each role there, algorithmic bytes from the Llama-3-8B shapes here."""
    rec = profile_record("decode_bs1_llama3_8b_q4_0")
    if not rec or "roles" not in rec:
        return None
    h, f, kvd, v = L3["hidden"], L3["ffn"], L3["kv_heads"] * 128, L3["vocab"]
    q40 = lambda n, k: n * k * 18 // 32
    ctx = rec.get("mean_ctx", prompt_len)
    algo = {
        "qkv": q40(h + 2 * kvd, h) + 4 * h + 4 * h + 2 * 2 * kvd,        # weights, f32 x + gamma, K/V append
        "o_proj": q40(h, h) + 2 * h + 4 * h + 4 * h,                      # weights, f16 x, f32 resid in / out
        "gate_up": q40(2 * f, h) + 4 * h + 4 * h + 2 * f,
        "down": q40(h, f) + 2 * f + 4 * h + 4 * h,
        "attention": 2 * 2 * kvd * ctx + 4 * h + 2 * h,                 # K and V rows once, q in, out
        "lm_head": 2 * v * h + 4 * h + 4 * h + 4 * v,
    }
    out = {"source": "profiles/decode_bs1_llama3_8b_q4_0.md", "commit": rec.get("commit")}
    for role, us in rec["roles"].items():
        if role in algo:
            gbs = algo[role] / us / 1e3
            out[role] = {"us": round(us, 2), "bytes": algo[role], "GB_s": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-bs32", action="store_true")
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--no-c3", action="store_true")
    ap.add_argument("--only", choices=["all", "roofline", "bs1", "bs1pen", "bs1ref", "stream", "bs32", "copy", "attn", "c3", "gemm",
                                       "kquant"],
                    default="all",
                    help="run one section alone (for rocprofv3 runs); 'all' prints the JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (--gpus must be 1)", file=sys.stderr)
        return 2

    import torch
    from janus_amd import _lib, ops
    if not _lib.LIB_PATH.exists():
        from janus_amd import build
        build.build_library()
    engine = ops.ComputeEngine(0)

    if args.only == "copy":
        log(f"copy: {copy_bandwidth():.0f} GB/s (1 GiB device copy, read + write)")
        return 0
    attn = None
    if args.only in ("all", "attn"):
        a_us, a_bytes, a_rows = attention_c4(engine)
        attn = {"us_per_launch": round(a_us, 2), "GB_s": round(a_bytes / a_us / 1e3, 1), "ctx_sum": a_rows,
                "algorithmic_bytes": a_bytes}
        log(f"attention C4: {a_us:.1f} us/launch, {a_bytes / a_us / 1e3:.0f} GB/s (ctx sum {a_rows})")
        if args.only == "attn":
            return 0
    gemm = None
    if args.only in ("all", "gemm"):
        gemm = {}
        for n, k in ((14336, 4096), (6144, 4096), (4096, 4096), (28672, 4096), (4096, 14336)):
            u, b, fl = gemm_m32(engine, n, k)
            gemm[f"{n}x{k}"] = {"us_per_launch": round(u, 2), "GB_s": round(b / u / 1e3, 1),
                                "TFLOP_s": round(fl / u / 1e6, 1), "mfma_frac": round(fl / u / 1e6 / MFMA_PEAK_TFLOPS, 4)}
            log(f"  Q4_0 GEMM M=32 {n}x{k}: {u:.2f} us, {b / u / 1e3:.0f} GB/s, {fl / u / 1e6:.0f} TFLOP/s "
                f"({fl / u / 1e6 / MFMA_PEAK_TFLOPS:.3f} of dense fp16 MFMA)")
        if args.only == "gemm":
            return 0
    kq = None
    if args.only in ("all", "kquant"):
        # K-quant products at the Llama-3-8B decode shapes (x fp16, y fp16)
        kq = {}
        for qname, qt in (("q4_k", 12), ("q5_k", 13)):
            for n, k in ((14336, 4096), (4096, 14336)):
                u, b, _ = gemv_roofline(engine, n, k, qtype=qt)
                kq[f"gemv_{qname}_{n}x{k}"] = {"us_per_launch": round(u, 3), "GB_s": round(b / u / 1e3, 1),
                                               "frac": round(b / u / 1e3 / HBM_PEAK_GBS, 4)}
                log(f"  {qname.upper()} GEMV {n}x{k}: {u:.2f} us/launch, {b / u / 1e3:.0f} GB/s "
                    f"({b / u / 1e3 / HBM_PEAK_GBS:.3f} of 8 TB/s)")
        u, b, fl = gemm_m32(engine, 14336, 4096, qtype=13)
        kq["gemm_m32_q5_k_14336x4096"] = {"us_per_launch": round(u, 2), "GB_s": round(b / u / 1e3, 1),
                                          "TFLOP_s": round(fl / u / 1e6, 1),
                                          "mfma_frac": round(fl / u / 1e6 / MFMA_PEAK_TFLOPS, 4)}
        log(f"  Q5_K GEMM M=32 14336x4096: {u:.2f} us, {b / u / 1e3:.0f} GB/s, {fl / u / 1e6:.0f} TFLOP/s")
        if args.only == "kquant":
            return 0
    if args.only in ("all", "roofline"):
        log("roofline: Q4_0 GEMV 14336x4096")
        us, algo, copies = gemv_roofline(engine)
        achieved = algo / us / 1e3
        log(f"  {us:.2f} us/launch, {achieved:.0f} GB/s over {copies} weight copies")
        if args.only == "roofline":
            return 0
    if args.only == "all":
        shapes = {}
        for n, k in ((4096, 14336), (4096, 4096)):
            u2, a2, _ = gemv_roofline(engine, n, k)
            shapes[f"{n}x{k}"] = {"us_per_launch": round(u2, 3), "GB_s": round(a2 / u2 / 1e3, 1)}
            log(f"  Q4_0 GEMV {n}x{k}: {u2:.2f} us/launch, {a2 / u2 / 1e3:.0f} GB/s")
        copy_gbs = copy_bandwidth()
        log(f"  device copy: {copy_gbs:.0f} GB/s")

    c3 = None
    if args.only in ("all", "c3") and not args.no_c3:
        log("config 3: building Llama-2-7B-shape Q4_K model (random init, shared layer bytes)")
        t0 = time.time()
        spec2 = llama2_q4k_spec(3, args.layers)
        log(f"  synthesised in {time.time() - t0:.1f} s")
        ms3, n3, pre_s = decode_c3(engine, spec2)
        c3 = {"tok_s": round(n3 / (ms3 / 1e3), 1), "ms_per_token": round(ms3 / n3, 4), "decode_tokens": n3,
              "prompt": 512, "ctx": 2048, "prefill_s": round(pre_s, 2)}
        log(f"config 3 Llama-2-7B Q4_K: {ms3 / n3:.3f} ms/token, {c3['tok_s']} tok/s over {n3} decode tokens "
            f"(context 513-2048)")
        del spec2
        if args.only == "c3":
            return 0

    log("building Llama-3-8B-shape Q4_0 model (random init)")
    t0 = time.time()
    spec = llama3_spec(7, args.layers)
    log(f"  synthesised in {time.time() - t0:.1f} s")
    if args.only == "bs32":
        ms32, ctx_sum = decode_bs32(engine, spec, args.steps, args.warmup)
        log(f"bs=32 ragged: {ms32 / args.steps:.3f} ms/step, {32 * args.steps / (ms32 / 1e3):.1f} tok/s")
        return 0
    if args.only == "bs1ref":
        nref = max(10, args.steps // 4)
        msr, _ = decode_bs1(engine, spec, nref, args.warmup, f32=True)
        log(f"bs=1 reference dtypes: {msr / nref:.3f} ms/token")
        return 0
    if args.only == "stream":
        mss, nst = decode_stream(engine, spec)
        log(f"bs=1 streaming: {mss:.3f} ms/token (median callback interval over {nst} tokens)")
        return 0
    if args.only == "bs1pen":
        msp, _ = decode_bs1(engine, spec, args.steps, args.warmup, penalty=1.15, trials=HEADLINE_TRIALS)
        log(f"bs=1 penalty 1.15: {msp / args.steps:.3f} ms/token")
        return 0
    # the headline: W warmup steps, then 5 timed runs of exactly K steps each
    # (each bracketed by device synchronisation); the median run is reported
    ms, toks = decode_bs1(engine, spec, args.steps, args.warmup, trials=HEADLINE_TRIALS)
    tok_s = args.steps / (ms / 1e3)
    log(f"bs=1: {ms / args.steps:.3f} ms/token, {tok_s:.1f} tok/s (median of {HEADLINE_TRIALS} runs of "
        f"{args.steps} timed steps)")
    if args.only == "bs1":
        return 0
    msp, _ = decode_bs1(engine, spec, args.steps, args.warmup, penalty=1.15)
    bs1_pen = {"tok_s": round(args.steps / (msp / 1e3), 2), "ms_per_token": round(msp / args.steps, 4),
               "sampler": "repetition penalty 1.15 over the generated tokens + last-max argmax, in the captured step"}
    log(f"bs=1 penalty 1.15: {msp / args.steps:.3f} ms/token, {bs1_pen['tok_s']} tok/s")
    msr, _ = decode_bs1(engine, spec, max(10, args.steps // 4), args.warmup, f32=True)
    nref = max(10, args.steps // 4)
    bs1_ref = {"tok_s": round(nref / (msr / 1e3), 2), "ms_per_token": round(msr / nref, 4),
               "dtypes": "f32 activations into the products, f32 KV (the reference's), plain argmax"}
    log(f"bs=1 reference dtypes: {msr / nref:.3f} ms/token, {bs1_ref['tok_s']} tok/s")
    mss, nst = decode_stream(engine, spec)
    bs1_stream = {"ms_per_token": round(mss, 4), "tok_s": round(1e3 / mss, 2), "tokens": nst,
                  "how": "janus_model_generate_stream with penalty 1.15: median interval between consecutive "
                         "per-token callbacks (host wall clock)"}
    log(f"bs=1 streaming: {mss:.3f} ms/token over {nst} tokens")

    bs32 = None
    if not args.no_bs32:
        steps32 = max(10, args.steps // 10)
        ms32, ctx_sum = decode_bs32(engine, spec, steps32, 3)
        bs32 = {"tok_s": round(32 * steps32 / (ms32 / 1e3), 1), "ms_per_step": round(ms32 / steps32, 3),
                "steps": steps32, "ctx_sum": ctx_sum}
        log(f"bs=32 ragged: {ms32 / steps32:.3f} ms/step, {bs32['tok_s']} tok/s")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline: oracle, OpenMP over rows, 20 decode tokens")
        v, threads, dt = cpu_baseline(spec)
        cpu = {"value": round(v, 4), "unit": "tok/s", "cores": threads, "kind": "port",
               "sample": f"20 greedy decode tokens (positions 0-19) of the same Llama-3-8B-shape Q4_0 model "
                         f"through the C oracle (a restatement of the reference arithmetic, not the reference), "
                         f"products OpenMP over rows on {threads} threads; median token time of the 20, "
                         f"{dt:.1f} s in all"}
    in_step = in_step_fractions()
    rec = profile_record("gemv_q4_0_14336x4096_f16") or {}

    line = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "trials": HEADLINE_TRIALS, "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (random-init weights, seeded prompt)",
        "config": {"workload": "Llama-3-8B-shape Q4_0 greedy decode, batch 1, 128-token prompt, fp16 KV, "
                               "F16 LM head, HIP-graph decode step, model at the 8192-token context",
                   "layers": args.layers,
                   "hidden": 4096, "heads": 32, "kv_heads": 8, "ffn": 14336, "vocab": 128256},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": rec.get("traffic_bytes"),
                     "traffic_source": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE per launch, scaled by a "
                                       "device copy's counts (profiles/gemv_q4_0_14336x4096_f16.md, commit "
                                       f"{rec.get('commit')})",
                     "kernel": "Q4_0 GEMV 14336x4096 (x fp16, y fp16)", "us_per_launch": round(us, 3),
                     "algorithmic_bytes": algo, "other_shapes": shapes, "device_copy_GB_s": round(copy_gbs, 1)},
        "bs32": bs32,
        "bs1_penalty": bs1_pen,
        "bs1_reference_dtype": bs1_ref,
        "bs1_stream": bs1_stream,
        "in_step": in_step,
        "gemm_m32_q4_0": gemm,
        "kquant": kq,
        "llama2_7b_q4k_c3": c3,
        "attention_c4": attn,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    engine.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
