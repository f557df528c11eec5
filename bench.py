#!/usr/bin/env python3
"""Benchmark of the brain step on one MI355X: the Seoul-shaped greedy decode (B=1 and the two-conversation step,
B=2), the roofline of its dominant kernel, and imi's CPU path (the oracle restatement) timed on the host cores.

    python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--cpu-threads N] [--no-cpu]

Prints one JSON line. A step is one decode position of the Seoul-shaped model (16 layers: 10 gated short-conv blocks,
6 GQA blocks 32/8 x 64, FFN 8192, tied Q4_0 word table 97,496 x 2048), synthetic seeded weights, a 32-token seeded
prompt, then --steps greedy ids generated on the device (argmax fed back without host round trips), context 512.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
GATE_UP_TRAFFIC_BYTES = 19_302_765   # counters: 149,528 128-B + 1,525.7 64-B read requests + 64 KiB WRITE_SIZE per launch
# matrix-core utilisation of the prefill's table products, rocprofv3's MfmaUtil per dispatch (MFMA busy cycles over
# GUI-active cycles x SIMDs) from `rocprofv3 --pmc MfmaUtil --kernel-include-regex k_pf_ -- python3 bench.py
# --prefill-only --prefill-reps 2`: a counter run, not measurable from inside this process
PREFILL_MFMA_UTIL_PCT = {"ffn_gate_up k_pf_gemm_lds<1,false,4,32>": 30.7, "in_proj k_pf_gemm_lds<0,false,4,32>": 19.5,
                         "2048-row tables k_pf_gemm_lds<0,false,4,16>": 20.8,
                         "q|k|v|gate k_pf_gemm_lds<0,false,4,16>": 20.5}
N_CTX = 512
PROMPT = 32


def _prompt(seed, vocab):
    return np.random.default_rng(seed).integers(0, vocab, size=PROMPT).astype(np.int32)


def gpu_decode(brain, steps, warmup, b2: bool):
    """Greedy decode after the prompt; returns (tokens/s over the timed steps, ids, device seconds)."""
    def prepare():
        sa = brain.new_state()
        sb = brain.new_state() if b2 else None
        pa, pb = _prompt(0, brain.n_vocab), _prompt(1, brain.n_vocab)
        for i in range(PROMPT):
            last = i == PROMPT - 1
            if b2:
                (_, _, ba), (_, _, bb) = brain.step2(int(pa[i]), None, last, sb, int(pb[i]), None, last, a=sa)
            else:
                _, _, ba = brain.step(int(pa[i]), want_logits=last, st=sa)
                bb = None
        return sa, sb, ba, bb

    sa, sb, ba, bb = prepare()
    if warmup:
        brain.generate(ba, warmup, b=sb, first_b=bb or 0, a=sa)
    sa, sb, ba, bb = prepare()
    t0 = time.perf_counter()
    out = brain.generate(ba, steps, b=sb, first_b=bb or 0, a=sa)
    wall = time.perf_counter() - t0
    ids, dev = ((out[0], out[1]), out[2]) if b2 else out
    tokens = steps * (2 if b2 else 1)
    return tokens / wall, ids, dev, wall


def _progress(msg):
    """One line on stderr as each part of the run ends (the JSON result stays alone on stdout)."""
    print(f"bench.py: {msg}", file=sys.stderr, flush=True)


def real_seoul_decode(steps, warmup):
    """Greedy decode on the shape of the released Seoul files (24 layers, 16/4 x 128 heads, FFN 7680, 7-tap conv,
    rope_freqs, window 256 on 4 of the 8 attention layers, Q6_K tied word table), B=1 and B=2."""
    import nunchi_amd
    from nunchi_amd import synth
    shp = synth.REAL_SEOUL
    rb = nunchi_amd.Brain(synth.cached("brain", shp, 0), n_ctx=N_CTX)
    t1, _, d1, _ = gpu_decode(rb, steps, warmup, b2=False)
    t2, _, d2, _ = gpu_decode(rb, steps, warmup, b2=True)
    # algorithmic bytes of a step: every table once, the fp32 vectors, the K and V rows the attention layers read
    # (window layers at most 256 positions), averaged over the generated positions
    kv_head = rb.n_head_kv * rb.head_dim * 2
    n_full = rb.n_attn - len(shp.swa_layers)
    kv = sum(2 * kv_head * (n_full * (PROMPT + i + 1) + len(shp.swa_layers) * min(PROMPT + i + 1, shp.sliding_window))
             for i in range(steps)) / steps
    step_b = rb.table_bytes + rb.vector_bytes + kv
    out = {"workload": "Seoul file shape: 24 layers (16 short-conv k=7, 8 GQA 16/4 x 128 with q/k norms and gates, "
                       "rope_freqs divisors, window 256 on layers 2/8/14/20), FFN 7680, tied Q6_K vocab 97496 x 2048, "
                       f"fp16 KV ctx {N_CTX}; {PROMPT}-token seeded prompt then {steps} greedy ids on device",
           "b1_tokens_per_s": round(t1, 1), "b2_tokens_per_s": round(t2, 1),
           "device_ms_per_step": {"b1": round(d1 * 1e3 / steps, 4), "b2": round(d2 * 1e3 / steps, 4)},
           "bytes_per_step": int(step_b),
           "hbm_fraction": {"b1": round(step_b * t1 / 1e9 / HBM_PEAK_GBS, 4), "b2": round(step_b * t2 / 2 / 1e9 / HBM_PEAK_GBS, 4)}}
    del rb
    return out


def cpu_decode(path, threads, steps, b2: bool, runs: int = 1):
    """imi's CPU path (the oracle restatement): `runs` conversations, each a 32-token prompt then `steps` greedy
    ids; returns (tokens/s over the generated tokens of all runs, ids of run 0 (B=2: both conversations'), seconds)."""
    import oracle
    eng = oracle.Engine(path, threads=threads, n_ctx=N_CTX)
    tok, secs, ids0 = 0, 0.0, None
    for r in range(runs):
        eng.reset()
        pa, pb = _prompt(2 * r, eng.n_vocab), _prompt(2 * r + 1, eng.n_vocab)
        if b2:
            sb = eng.new_state()
            for i in range(PROMPT):
                last = i == PROMPT - 1
                _, la, _, lb = eng.step2(int(pa[i]), None, last, sb, int(pb[i]), None, last)
            oa, ob, t = eng.greedy2(sb, oracle.top(la), oracle.top(lb), steps)
            oa = (oa, ob)
            tok += 2 * steps
        else:
            for i in range(PROMPT):
                _, lg = eng.step(int(pa[i]), want_logits=i == PROMPT - 1)
            oa, t = eng.greedy(oracle.top(lg), steps)
            tok += steps
        secs += t
        if ids0 is None:
            ids0 = oa
    return tok / secs, ids0, secs


VOICE_CTX = 4096      # slot A's KV context in the voice frame
VOICE_WARMUP = 4      # untimed frames before the timed ones (slot B starts at position 0)
A_POS = 2048          # slot A's position when the timed frames start
SCHEDULE = (4, 4)     # masked passes of a frame: codebooks scored (and fixed) by each, in a shuffled order
TALK_SCHEDULE = (6, 6)   # imi's schedule for its 12 codebooks (imi/core/talk.cpp:129)
TEMP, REP, REP_WIN = 0.4, 1.2, 64   # imi's sampling settings (imi/core/talk.cpp:131-133)


def play_frames(step2, voice, tok_a, fb, frames, pick, schedule=SCHEDULE, codec=None):
    """Voice frames as imi's talk loop runs them (imi/core/talk.cpp:127-187) with slot A riding along
    (imi/core/flow.cpp:118): step2 (A: text step with scores, B: the voice brain step fed the last feedback row sum),
    begin_frame from B's hidden state, the masked passes over a shuffled codebook order (each samples its
    codebooks' codes with temperature 0.4 and repeat penalty 1.2 over the last 64 frames: `pick` runs the pass
    and the sampling), then the codec turns the codes into the frame's samples (imi/core/talk.cpp:178-180) and the
    feedback row sum is formed. The shuffles and uniform draws come from one seeded generator (numpy's, in place of
    imi's mt19937), so two runs with the same scores pick the same codes; an end-of-audio pick does not end the run,
    and codes past the codec's level table (the end-of-audio and other special codes, which end a real run) are
    wrapped into it so every frame is decoded. Returns per-frame seconds, the step2 and generator shares, the codes of
    every frame, slot A's ids, and the codec's shares and samples."""
    tot, br, vo, codes_all, ids, cd, pcm = [], [], [], [], [], [], []
    rng = np.random.default_rng(7)
    for _ in range(frames):
        order = rng.permutation(voice.n_cb).astype(np.int32)
        u = rng.uniform(size=voice.n_cb)
        window = np.array(codes_all[-REP_WIN:], np.int32).reshape(-1, voice.n_cb)
        t0 = time.perf_counter()
        tok_a, hb = step2(tok_a, fb)
        t1 = time.perf_counter()
        voice.begin_frame(hb)
        codes = np.full(voice.n_cb, -1, np.int32)
        k = 0
        for n in schedule:
            need = order[k:k + n]
            codes[need] = pick(voice, codes, need, window, u[k:k + n])
            k += n
        t2 = time.perf_counter()
        if codec is not None:
            pcm.append(codec.frame(codes % codec_levels(codec)))
        t3 = time.perf_counter()
        fb = voice.feedback(codes)
        t4 = time.perf_counter()
        tot.append(t4 - t0)
        br.append(t1 - t0)
        vo.append((t2 - t1) + (t4 - t3))
        cd.append(t3 - t2)
        codes_all.append(codes)
        ids.append(tok_a)
    return (np.array(tot), np.array(br), np.array(vo), np.array(codes_all), ids, tok_a, fb, np.array(cd),
            np.concatenate(pcm) if pcm else np.zeros(0, np.float32))


def codec_levels(codec) -> int:
    """Rows of the codec's FSQ level table (the codes it takes)."""
    return codec.info.n_codes if hasattr(codec, "info") else codec.n_codes


def gpu_voice_frames(brain_path, voice_path, frames, warmup, a_pos=A_POS, schedule=SCHEDULE, codec_path=None):
    """Voice frames on the device: slot A decodes greedily to position a_pos first, then the frames run."""
    import nunchi_amd
    brain = nunchi_amd.Brain(brain_path, n_ctx=VOICE_CTX)
    voice = nunchi_amd.Voice(voice_path)
    codec = nunchi_amd.Codec(codec_path) if codec_path else None
    sa, sb = brain.new_state(), brain.new_state()
    pa = _prompt(2, brain.n_vocab)
    for i in range(PROMPT):
        _, _, ba = brain.step(int(pa[i]), want_logits=i == PROMPT - 1, st=sa)
    ids = brain.generate(ba, a_pos - PROMPT, a=sa)[0] if a_pos > PROMPT else np.array([ba], np.int32)

    def step2(tok, fb):
        (_, _, best), (hb, _, _) = brain.step2(tok, None, True, sb, -1, fb, False, a=sa)
        return best, hb

    fb = voice.feedback(np.zeros(voice.n_cb, np.int32))
    ref = play_frames(step2, voice, int(ids[-1]), fb, frames + warmup,
                      lambda v, codes, need, win, u: (v.pass_(codes, need, scores=False),
                                                      v.sample(win, u, TEMP, REP)[0])[1], schedule, codec)
    # the timed frames are the frames after the warmup ones, in the same run (states keep advancing)
    out = tuple(x[warmup:] for x in ref[:4]) + (ref[4][warmup:], ref[7][warmup:])
    info = {"table_bytes": voice.table_bytes, "n_cb": voice.n_cb}
    if codec is not None:
        info["codec_table_bytes"] = int(codec.info.table_bytes)
        codec.close()
    voice.close()
    brain.ctx.close()
    return out, ref, info


def cpu_voice_frames(brain_path, voice_path, threads, frames, a_pos=A_POS, schedule=SCHEDULE, codec_path=None):
    import oracle
    eng = oracle.Engine(brain_path, threads=threads, n_ctx=VOICE_CTX)
    voice = oracle.Voice(voice_path, threads=threads)
    codec = oracle.Codec(codec_path) if codec_path else None
    pa = _prompt(2, eng.n_vocab)
    for i in range(PROMPT):
        _, lg = eng.step(int(pa[i]), want_logits=i == PROMPT - 1)
    ids = eng.greedy(oracle.top(lg), a_pos - PROMPT)[0] if a_pos > PROMPT else np.array([oracle.top(lg)], np.int32)
    st = eng.new_state()

    def step2(tok, fb):
        _, la, hb, _ = eng.step2(tok, None, True, st, -1, fb, False)
        return oracle.top(la), hb

    fb = voice.feedback(np.zeros(voice.n_cb, np.int32))
    return play_frames(step2, voice, int(ids[-1]), fb, frames,
                       lambda v, codes, need, win, u: oracle.voice_sample(v.pass_(codes, need), need, win, u, TEMP,
                                                                          REP)[0], schedule, codec)


HEAR_EMB, HEAR_TOK = 384, 64   # the hearing window: audio-encoder rows, then words


def hearing_inputs(vocab):
    rng = np.random.default_rng(12)
    emb = rng.standard_normal((HEAR_EMB + HEAR_TOK, 2048)).astype(np.float32)
    toks = np.full(HEAR_EMB + HEAR_TOK, -1, np.int32)
    toks[HEAR_EMB:] = np.random.default_rng(13).integers(0, vocab, size=HEAR_TOK)
    return toks, emb


def gpu_prefill(brain, reps):
    """The hearing window as one causal prefill (step_batch) on a fresh conversation; returns the wall seconds of
    each rep (inputs copied from the host inside the call), the last scores and the chosen id."""
    toks, emb = hearing_inputs(brain.n_vocab)
    st = brain.new_state()
    times = []
    for r in range(reps + 1):
        st.reset()
        t0 = time.perf_counter()
        _, lg, best, _ = brain.step_batch(toks, emb, want_logits=True, st=st)
        if r:
            times.append(time.perf_counter() - t0)
    return np.array(times), lg, best


HEAR_SAMPLES = 491760   # 30.7 s at 16 kHz: the ears give exactly the hearing window's 384 rows


def ears_fma(info, n_pos, n_fr):
    """fp32 multiply-adds of one encode (imi/core/ears.cpp:198-407): the DFT table, the three 3x3 convolutions, the
    pointwise and pre_encode tables, every layer's tables, conv taps and attention (scores and weighted values over
    the window), the projector; the mel filters' double multiply-adds are not counted."""
    C, E, F8, F2, F4 = info.n_ch, info.n_embd, info.n_mel // 8, info.n_mel // 2, info.n_mel // 4
    T2 = (n_fr + 1) // 2
    T4 = (T2 + 1) // 2
    H, Hk, D = info.n_head, info.n_head_kv, info.head_dim
    f = 402 * 400 * n_fr + 9 * C * (T2 * F2 + T4 * F4 + n_pos * F8) + C * C * (T4 * F4 + n_pos * F8) + E * C * F8 * n_pos
    n_conv = info.n_layer - info.n_attn
    keys = sum(min(p + 1, info.window) for p in range(n_pos))
    f += n_conv * ((3 * E * E + E * E + info.d_conv * E) * n_pos)
    f += info.n_attn * (((H + 2 * Hk) * D * E + E * H * D) * n_pos + 2 * H * D * keys)
    f += info.n_layer * 3 * info.n_ff * E * n_pos
    f += (info.n_mid * E + info.n_out * info.n_mid) * n_pos
    return f


def gpu_hear(brain, ears_path, reps):
    """The hearing window from sound: the ears encode a 30.7 s clip into 384 rows, then the rows and 64 seeded words
    run as one causal prefill. Returns per-rep ears and prefill seconds (host buffers in and out, as imi's caller
    passes them), the rows, the last scores and the chosen id."""
    import nunchi_amd
    from nunchi_amd import synth
    ears = nunchi_amd.Ears(ears_path)
    pcm = synth.clip(HEAR_SAMPLES, 1)
    toks, emb = hearing_inputs(brain.n_vocab)
    st = brain.new_state()
    te, tp = [], []
    for r in range(reps + 1):
        st.reset()
        t0 = time.perf_counter()
        rows = ears.encode(pcm)
        t1 = time.perf_counter()
        emb[:HEAR_EMB] = rows
        _, lg, best, _ = brain.step_batch(toks, emb, want_logits=True, st=st)
        t2 = time.perf_counter()
        if r:
            te.append(t1 - t0)
            tp.append(t2 - t1)
    info = ears.info
    ears.close()
    return np.array(te), np.array(tp), rows, lg, best, info


def cpu_hear(path, ears_path, threads):
    import oracle
    from nunchi_amd import synth
    pcm = synth.clip(HEAR_SAMPLES, 1)
    ears = oracle.Ears(ears_path, threads=threads)
    rows = ears.encode(pcm)
    rows = ears.encode(pcm)
    te = ears.secs
    del ears   # its spinning thread team would compete with the engine's
    toks, emb = hearing_inputs(97496)
    emb[:HEAR_EMB] = rows
    eng = oracle.Engine(path, threads=threads, n_ctx=N_CTX)
    t0 = time.perf_counter()
    _, lg, _ = eng.step_batch(toks, emb, want_logits=True)
    return te, time.perf_counter() - t0, rows, lg


def oracle_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.sqrt(((a - b) ** 2).sum() / max((b ** 2).sum(), 1e-30))


def cpu_prefill(path, threads):
    import oracle
    toks, emb = hearing_inputs(97496)
    eng = oracle.Engine(path, threads=threads, n_ctx=N_CTX)
    t0 = time.perf_counter()
    _, lg, _ = eng.step_batch(toks, emb, want_logits=True)
    return time.perf_counter() - t0, lg


def cpu_info():
    """The host CPU as this process sees it: model name, logical CPUs in the affinity mask, the physical cores they
    sit on and the SMT width (logical CPUs per core)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), model)
    except OSError:
        pass
    aff = sorted(os.sched_getaffinity(0))
    cores, smt = set(), 1
    for c in aff:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f1, open(base + "core_id") as f2:
                cores.add((f1.read().strip(), f2.read().strip()))
            with open(base + "thread_siblings_list") as f3:
                sib = f3.read().strip()
            smt = max(smt, sum(int(b) - int(a) + 1 if "-" in x else 1
                               for x in sib.split(",") for a, b in [x.split("-") if "-" in x else (x, x)]))
        except OSError:
            pass
    return {"model": model, "logical_cpus": len(aff), "physical_cores": len(cores) or None, "smt_width": smt}


# one Seoul-shaped layer's linears (rows, cols), imi's table order: q, k, v, o, gate, up, down
LAYER_TABLES = ((2048, 2048), (512, 2048), (512, 2048), (2048, 2048), (8192, 2048), (8192, 2048), (2048, 8192))
LAYER_COPIES = 16   # distinct device copies in rotation: 16 x 34.2 MB, more than the 256 MB MALL holds


def layer_weights():
    from nunchi_amd import synth
    rng = np.random.default_rng(300)
    w = [synth.q4_0_random(rng, r, c) for r, c in LAYER_TABLES]
    x = np.random.default_rng(301).standard_normal((2, 8192)).astype(np.float32)
    return w, x


def gpu_layer(ctx, reps):
    """cfg 1 on the device: the layer's 7 tables through the kernel-level GEMV (imi's int8 cut per 32 columns),
    LAYER_COPIES copies in rotation, one launch per table and grouped (sh_q4_gemv_group: the six 2048-wide tables in
    one launch, down in another); returns per-layer microseconds at B=1 and B=2 for both, the B=2 outputs of copy 0,
    and whether the grouped outputs equal the per-table ones bit for bit."""
    import nunchi_amd
    w, x = layer_weights()
    nt = len(LAYER_TABLES)
    tabs = [nunchi_amd.Q4Table(ctx, w[i], r, c) for _ in range(LAYER_COPIES) for i, (r, c) in enumerate(LAYER_TABLES)]
    out = [tabs[i].gemv(x[:, :c]) for i, (_, c) in enumerate(LAYER_TABLES)]
    grouped = nunchi_amd.q4_gemv_group(ctx, tabs[:nt], [x[:, :c] for _, c in LAYER_TABLES])
    same = all(np.array_equal(g.view(np.uint32), o.view(np.uint32)) for g, o in zip(grouped, out))
    us1 = nunchi_amd.q4_bench(ctx, tabs, n_in=1, cut_mode=0, reps=reps) * nt
    us2 = nunchi_amd.q4_bench(ctx, tabs, n_in=2, cut_mode=0, reps=reps) * nt
    sets = [tabs[k * nt:(k + 1) * nt] for k in range(LAYER_COPIES)]
    g1 = nunchi_amd.q4_group_bench(ctx, sets, n_in=1, cut_mode=0, reps=reps // nt)
    g2 = nunchi_amd.q4_group_bench(ctx, sets, n_in=2, cut_mode=0, reps=reps // nt)
    for t in tabs:
        t._free()
    return us1, us2, out, g1, g2, same


def cpu_layer(threads, seconds=2.0):
    """cfg 1 on the oracle (imi's group / group2 kernels on a `threads` team): per-layer microseconds at B=1 and
    B=2 (each table's fastest rep of enough reps for about `seconds` in all), and the B=2 outputs."""
    import oracle
    w, x = layer_weights()
    res, out = [], []
    for n_in in (1, 2):
        tot = 0.0
        for i, (r, c) in enumerate(LAYER_TABLES):
            t = oracle.Q4Table(w[i], r, c, threads=threads)
            y, s1 = t.gemv(x[:n_in, :c], reps=3)
            reps = max(3, int(seconds / len(LAYER_TABLES) / max(s1, 1e-6)))
            _, sec = t.gemv(x[:n_in, :c], reps=reps)   # the fastest rep
            tot += sec
            if n_in == 2:
                out.append(y)
            del t
        res.append(tot * 1e6)
    return res[0], res[1], out


def cpu_cfg0(threads, seconds=2.0):
    """cfg 0 on the oracle: imi/kernels/q4x8's GEMV 8192 x 2048, the fastest of about `seconds` of reps on one table
    (its figure of merit: table GB/s)."""
    import oracle
    from nunchi_amd import synth
    q = synth.q4_0_random(np.random.default_rng(100), 8192, 2048)
    x = np.random.default_rng(5).standard_normal(2048).astype(np.float32)
    t = oracle.Q4x8Table(q, 8192, 2048, threads=threads)
    _, s1 = t.gemv(x, reps=3)
    reps = max(3, int(seconds / max(s1, 1e-6)))
    _, sec = t.gemv(x, reps=reps)   # the fastest rep
    return 8192 * 64 * 18 / sec / 1e9


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--cpu-threads", type=int, default=0, help="0 = min(16, cores in the affinity mask)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=8, help="B=1 conversations timed on the CPU (B=2: half as many pairs)")
    ap.add_argument("--voice-frames", type=int, default=64, help="timed voice frames (cfg 4); 0 = skip")
    ap.add_argument("--prefill-reps", type=int, default=10, help="timed hearing-window prefills (cfg 3); 0 = skip")
    ap.add_argument("--cpu-voice-frames", type=int, default=8)
    ap.add_argument("--hear-reps", type=int, default=5, help="timed hearing windows from sound (ears + prefill); 0 = skip")
    ap.add_argument("--ears-only", type=int, default=0, metavar="REPS",
                    help="only REPS ears encodes of the 30.7 s clip (after one untimed), no brain: the launches a kernel "
                         "trace of the ears reads")
    ap.add_argument("--talk-frames", type=int, default=32, help="timed talk frames (12-codebook generator + codec); 0 = skip")
    ap.add_argument("--cpu-talk-frames", type=int, default=4)
    ap.add_argument("--decode-only", action="store_true",
                    help="only the decode runs and the in-step kernel timing (the launches a kernel trace of the step "
                         "should average), no CPU legs")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the hearing-window prefills (--prefill-reps timed after one untimed): the launches a "
                         "kernel trace or counter run of the prefill reads")
    ap.add_argument("--codec-only", type=int, default=0, metavar="FRAMES",
                    help="only FRAMES codec frames (seeded codes, after 4 untimed), no brain: the launches a kernel "
                         "trace of the codec reads")
    ap.add_argument("--floor-only", action="store_true",
                    help="only the cfg-0 GEMV (8192 x 2048 Q4_0, 64 copies in rotation) next to an empty dispatch and a "
                         "pure read of the same 9,437,184 bytes, each back to back: the launches a kernel trace of the "
                         "floor reads")
    ap.add_argument("--layer-only", action="store_true",
                    help="only cfg 1 (one layer's 7 linears through the kernel-level GEMV at B=1 and B=2, per table and "
                         "grouped, 16 copies in rotation): the launches a kernel trace of cfg 1 reads")
    ap.add_argument("--voice-only", type=int, default=0, metavar="FRAMES",
                    help="only cfg 4: FRAMES voice frames (step2 at KV context 2048+, generator passes of 4 + 4 with "
                         "sampling, after 4 untimed): the launches a kernel trace of the whole frame reads")
    ap.add_argument("--real-steps", type=int, default=128,
                    help="timed greedy ids on the Seoul file shape (24 layers, FFN 7680, Q6_K vocab); 0 = skip")
    ap.add_argument("--real-only", action="store_true", help="only the Seoul-file-shape decode")
    ap.add_argument("--counters-workload", action="store_true",
                    help="only the launches the hardware-counter runs read: a streaming kernel of known size (the "
                         "exponential over 16 Mi floats: 64 MiB read, 64 MiB written), 64 read-only GEMVs of known "
                         "size (8192 x 2048 Q4_0, 64 distinct copies: 9,437,184 table bytes each), 64 FFN gate|up "
                         "launches and two hearing-window prefills")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (conversations shard across "
              "GPUs with no exchange; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    if PROMPT + max(args.steps, args.warmup, args.real_steps) > N_CTX:
        print(f"bench.py: prompt + steps must fit the context of {N_CTX}", file=sys.stderr)
        sys.exit(2)

    import nunchi_amd
    from nunchi_amd import synth
    if args.floor_only:
        ctx = nunchi_amd.Context()
        copies = [nunchi_amd.Q4Table(ctx, synth.q4_0_random(np.random.default_rng(100 + i), 8192, 2048), 8192, 2048)
                  for i in range(64)]
        g_us = nunchi_amd.q4_bench(ctx, copies, n_in=1, cut_mode=1, reps=640)
        e_us = nunchi_amd.bench_empty(grid=1024, reps=1000)
        r_us, st = nunchi_amd.bench_read(9437184, copies=64, grid=1152, reps=640, stamps=True)
        # the decode step as if every launch were a pure read of its table: each table size read back to back from
        # HBM (enough copies in rotation to exceed the 256 MB MALL), times its launches per B=1 step, plus an empty
        # dispatch for each of the 6 attention launches and the end-of-step launch
        tables = {"ffn_gate_up": (16384 * 64 * 18, 16), "ffn_down": (2048 * 256 * 18, 16),
                  "conv_in_proj": (6144 * 64 * 18, 10), "o_out_proj": (2048 * 64 * 18, 16),
                  "qkvg": (3104 * 64 * 18, 6), "word_scores": (97496 * 64 * 18, 1)}
        reads = {}
        for name, (nbytes, _) in tables.items():
            copies = max(2, min(64, -(-600_000_000 // nbytes)))
            reads[name] = nunchi_amd.bench_read(nbytes, copies=copies, grid=max(256, nbytes // 8192),
                                                reps=max(64, min(640, int(2e9 // nbytes))))
        floor_us = sum(reads[k] * n for k, (_, n) in tables.items()) + 7 * e_us
        print(json.dumps({"floor_only": {"gemv_us": round(g_us, 3), "empty_kernel_us": round(e_us, 3),
                                         "pure_read_us": round(r_us, 3), "pure_read_last_start_us": round(st[0], 2),
                                         "pure_read_first_bytes_us": round(st[1], 2),
                                         "pure_read_last_end_us": round(st[2], 2),
                                         "step_table_reads_us": {k: round(v, 3) for k, v in reads.items()},
                                         "step_read_floor_us": round(floor_us, 1),
                                         "step_read_floor_tokens_per_s": round(1e6 / floor_us, 1)}}), flush=True)
        return
    if args.ears_only:
        ears = nunchi_amd.Ears(synth.cached("ears", synth.EARS, 3))
        pcm = synth.clip(HEAR_SAMPLES, 1)
        ts = []
        for i in range(args.ears_only + 1):
            t0 = time.perf_counter()
            ears.encode(pcm)
            if i:
                ts.append(time.perf_counter() - t0)
        print(json.dumps({"ears_only": {"reps": len(ts), "p50_ms": round(float(np.percentile(ts, 50)) * 1e3, 3),
                                        "table_bytes": int(ears.info.table_bytes)}}), flush=True)
        return
    if args.codec_only:
        codec = nunchi_amd.Codec(synth.cached("codec", synth.CODEC, 2))
        codes = np.random.default_rng(5).integers(0, codec.info.n_codes, (args.codec_only + 4, 12))
        ts = []
        for i, cc in enumerate(codes):
            t0 = time.perf_counter()
            codec.frame(cc)
            if i >= 4:
                ts.append(time.perf_counter() - t0)
        print(json.dumps({"codec_only": {"frames": len(ts), "p50_ms": round(float(np.percentile(ts, 50)) * 1e3, 3),
                                         "table_bytes": int(codec.info.table_bytes)}}), flush=True)
        return
    if args.real_only:
        print(json.dumps({"real_only": real_seoul_decode(max(1, args.real_steps), args.warmup)}), flush=True)
        return
    path = synth.cached("brain", synth.SEOUL, 0)
    if args.voice_only:
        vpath = synth.cached("voice", synth.VOICE, 1)
        (ft, fbr, fvo, _, _, _), _, vinfo = gpu_voice_frames(path, vpath, args.voice_only, VOICE_WARMUP)
        print(json.dumps({"voice_only": {"frames": int(len(ft)), "p50_ms": round(float(np.percentile(ft, 50)) * 1e3, 3),
                                         "step2_p50_ms": round(float(np.percentile(fbr, 50)) * 1e3, 3),
                                         "generator_p50_ms": round(float(np.percentile(fvo, 50)) * 1e3, 3)}}), flush=True)
        return
    brain = nunchi_amd.Brain(path, n_ctx=N_CTX)
    if args.layer_only:
        l_us1, l_us2, _, lg_us1, lg_us2, same = gpu_layer(brain.ctx, reps=16 * len(LAYER_TABLES) * 8)
        print(json.dumps({"layer_only": {"b1_us": round(l_us1, 2), "b2_us": round(l_us2, 2), "grouped_b1_us": round(lg_us1, 2),
                                         "grouped_b2_us": round(lg_us2, 2), "grouped_equal_per_table": bool(same)}}),
              flush=True)
        return
    if args.counters_workload:
        x = np.linspace(-10.0, 10.0, 16 << 20, dtype=np.float32)
        brain.ctx.expf(x)
        copies = [nunchi_amd.Q4Table(brain.ctx, synth.q4_0_random(np.random.default_rng(100 + i), 8192, 2048), 8192, 2048)
                  for i in range(64)]
        nunchi_amd.q4_bench(brain.ctx, copies, n_in=1, cut_mode=1, reps=64)
        rd = nunchi_amd.q4_bench_kernel(brain.ctx, copies, n_in=1, cut_mode=1, reps=64)
        for t in copies:
            t._free()
        gu = brain.bench_kernel("ffn_gate_up", n_in=1, reps=64)
        pt, _, _ = gpu_prefill(brain, 1)
        print(json.dumps({"counters_workload": {"copy_bytes_read": int(x.nbytes), "copy_bytes_written": int(x.nbytes),
                                                "read_gemv_table_bytes": 8192 * 64 * 18, "read_gemv_avg_us": round(rd, 3),
                                                "ffn_gate_up_avg_us": round(gu["avg_us"], 3),
                                                "ffn_gate_up_bytes_per_launch": int(gu["bytes_per_launch"]),
                                                "prefill_ms": round(float(pt.min()) * 1e3, 3)}}))
        return

    if args.prefill_only:
        pt, _, pbest = gpu_prefill(brain, max(1, args.prefill_reps))
        print(json.dumps({"prefill_only": {"reps": int(len(pt)), "best_ms": round(float(pt.min()) * 1e3, 3),
                                           "p50_ms": round(float(np.percentile(pt, 50)) * 1e3, 3), "best_id": int(pbest)}}),
              flush=True)
        return

    tok_s_b1, ids_b1, dev_b1, wall_b1 = gpu_decode(brain, args.steps, args.warmup, b2=False)
    tok_s_b2, ids_b2, dev_b2, wall_b2 = gpu_decode(brain, args.steps, args.warmup, b2=True)
    _progress(f"decode B=1 {tok_s_b1:.1f}, B=2 {tok_s_b2:.1f} tokens/s")
    # the dominant kernel as it runs inside the step: inputs just written by the step's previous kernel, tables from
    # HBM (16 launches per step over 32 steps)
    gu_step = brain.bench_step_kernel("ffn_gate_up", n_in=1, steps=32)
    if args.decode_only:
        print(json.dumps({"decode_only": {"b1_tokens_per_s": round(tok_s_b1, 1), "b2_tokens_per_s": round(tok_s_b2, 1),
                                          "ffn_gate_up_in_step_us": round(gu_step["avg_us"], 3),
                                          "launches": gu_step["launches"]}}), flush=True)
        return

    # the per-table kernels (the same stages as separate launches; the step kernel's fallback path)
    gu = brain.bench_kernel("ffn_gate_up", n_in=1, reps=64)
    dn = brain.bench_kernel("ffn_down", n_in=1, reps=64)
    ws = brain.bench_kernel("word_scores", n_in=1, reps=8)
    gu2 = brain.bench_kernel("ffn_gate_up", n_in=2, reps=64)
    tables1 = brain.bench_tables(1, 5)
    tables2 = brain.bench_tables(2, 5)
    # imi's own word-table format: the same vocab shape as Q6_K (one layer in front, only the scores are timed)
    q6_shape = synth.BrainShape(n_layer=1, attn_layers=(), n_vocab=synth.SEOUL.n_vocab, vocab_type="q6_k")
    q6_brain = nunchi_amd.Brain(synth.cached("brain", q6_shape, 0), n_ctx=64)
    ws6 = q6_brain.bench_kernel("word_scores", n_in=1, reps=8)
    ws6_2 = q6_brain.bench_kernel("word_scores", n_in=2, reps=8)
    del q6_brain

    _progress("per-table kernels timed")
    # cfg 0: one Q4_0 x fp32 GEMV 8192 x 2048 with imi/kernels/q4x8 semantics, 64 distinct weight copies in rotation
    ctx = brain.ctx
    copies = [nunchi_amd.Q4Table(ctx, synth.q4_0_random(np.random.default_rng(100 + i), 8192, 2048), 8192, 2048) for i in range(64)]
    cfg0_us = nunchi_amd.q4_bench(ctx, copies, n_in=1, cut_mode=1, reps=640)           # per call, back to back
    cfg0_graph_us = nunchi_amd.q4_bench_graph(ctx, copies, n_in=1, cut_mode=1, passes=10)  # replayed from a graph
    cfg0_kernel_us = nunchi_amd.q4_bench_kernel(ctx, copies, n_in=1, cut_mode=1, reps=256)   # the kernel itself
    cfg0_bytes = 8192 * 64 * 18 + 2048 * 4 + 8192 * 4
    del copies
    # cfg 1: one layer's linears, B=1 and B=2 (two inputs riding each table read)
    l_us1, l_us2, l_out, lg_us1, lg_us2, l_group_same = gpu_layer(ctx, reps=16 * len(LAYER_TABLES) * 8)
    layer_bytes = sum(r * c // 32 * 18 for r, c in LAYER_TABLES)

    gu_gbs = gu["bytes_per_launch"] / (gu["avg_us"] * 1e-6) / 1e9
    gs_gbs = gu_step["bytes_per_launch"] / (gu_step["avg_us"] * 1e-6) / 1e9
    # algorithmic bytes of a decode step: every table once (device layout = file bytes: 16 B codes + 2 B scale per
    # 32 weights), the fp32 norm / conv vectors, and the K and V rows the step's attention reads (positions 0..pos of
    # n_attn layers x n_kv heads x D, fp16), averaged over the generated positions
    kv_row = brain.n_attn * brain.n_head_kv * brain.head_dim * 2
    vec_bytes = brain.vector_bytes
    gen_bytes = sum(brain.table_bytes + vec_bytes + 2 * kv_row * (PROMPT + i + 1) for i in range(args.steps))
    step_bytes = gen_bytes / args.steps
    # what the dispatch path and HBM allow a kernel reading the cfg-0 table's bytes: an empty 1024 x 256 kernel and a
    # pure read of 9,437,184 bytes (64 copies in rotation: every launch from HBM), each back to back on one stream
    e_us = nunchi_amd.bench_empty(grid=1024, reps=1000)
    r_us, r_st = nunchi_amd.bench_read(9437184, copies=64, grid=1152, reps=256, stamps=True)
    cfg0_floor = {"empty_kernel_us": round(e_us, 3), "pure_read_us": round(r_us, 3),
                  "pure_read_timeline_us": {"last_wg_start": round(r_st[0], 2), "first_bytes_p50": round(r_st[1], 2),
                                            "last_wg_end": round(r_st[2], 2)},
                  "pure_read_GBs": round(9437184 / r_us / 1e3, 1), "pure_read_frac": round(9437184 / r_us / 1e3 / HBM_PEAK_GBS, 4),
                  "gemv_over_pure_read": round(cfg0_us / r_us, 3)}
    line = {
        "metric": "brain-step tokens/s (B=1,2) + Q4_0 GEMV HBM GB/s vs roofline, 1 MI355X",
        "value": round(tok_s_b1, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 / tok_s_b1, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 x q4_0 -> int32 dots, fp32 epilogue",
        "data": "synthetic (seeded random Q4_0 weights of the Seoul shape)",
        "config": {
            "workload": "cfg2: Seoul-shaped brain decode, 16 layers (10 short-conv k=3, 6 GQA 32/8 x 64, RoPE 1e6), FFN 8192, "
                        "tied Q4_0 vocab 97496 x 2048, fp16 KV ctx 512; 32-token seeded prompt then greedy ids on device",
            "batch": 1,
            "generated_tokens": args.steps,
            "prompt_tokens": PROMPT,
        },
        "b2_tokens_per_s": round(tok_s_b2, 1),
        "b2_ms_per_step": round(2e3 / tok_s_b2, 4),
        "device_ms_per_step": {"b1": round(dev_b1 * 1e3 / args.steps, 4), "b2": round(dev_b2 * 1e3 / args.steps, 4)},
        "step_hbm_fraction": {"b1": round(step_bytes * tok_s_b1 / 1e9 / HBM_PEAK_GBS, 4),
                              "b2": round(step_bytes * tok_s_b2 / 2 / 1e9 / HBM_PEAK_GBS, 4),
                              "bytes_per_step": int(step_bytes)},
        # the dominant kernel of the step: FFN gate|up (16 launches per step, the largest share of its time), timed
        # inside whole steps (events of each launch's own dispatch on the context's stream, 512 launches)
        "roofline": {
            "kernel": "k_gemv_norm<1, EPI_SWIGLU, 2> (FFN gate|up 16384 x 2048 Q4_0 with the post-norm residual, RMS "
                      "norm, int8 cut and SwiGLU fused; B=1)",
            "bound": "hbm",
            "achieved": round(gs_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gs_gbs / HBM_PEAK_GBS, 4),
            # HBM bytes per launch from the FETCH_SIZE / WRITE_SIZE counter runs of `bench.py --counters-workload`,
            # calibrated on a streaming kernel and a read-only GEMV of known sizes
            "traffic": GATE_UP_TRAFFIC_BYTES,
            "traffic_source": "counter run (not this process): profiles/ffn_gate_up_counters_seoul.md",
            "launch_us": round(gu_step["avg_us"], 3),
            "launches_timed": gu_step["launches"],
            "bytes_per_launch": int(gu_step["bytes_per_launch"]),
            "isolated_launch_us": round(gu["avg_us"], 3),
            "isolated_frac": round(gu_gbs / HBM_PEAK_GBS, 4),
        },
        "kernels": {
            "ffn_gate_up_per_table": {"avg_us": round(gu["avg_us"], 3), "GBs": round(gu_gbs, 1), "frac": round(gu_gbs / HBM_PEAK_GBS, 4)},
            "ffn_gate_up_b2": {"avg_us": round(gu2["avg_us"], 3), "GBs": round(gu2["bytes_per_launch"] / gu2["avg_us"] / 1e3, 1)},
            "ffn_down": {"avg_us": round(dn["avg_us"], 3), "GBs": round(dn["bytes_per_launch"] / dn["avg_us"] / 1e3, 1)},
            # (back-to-back launches of one table: it fits the 256 MB MALL, so these read faster than a decode step's)
            "word_scores": {"avg_us": round(ws["avg_us"], 3), "GBs": round(ws["bytes_per_launch"] / ws["avg_us"] / 1e3, 1)},
            "word_scores_q6k_97496x2048": {"avg_us": round(ws6["avg_us"], 3), "GBs": round(ws6["bytes_per_launch"] / ws6["avg_us"] / 1e3, 1),
                                           "b2_avg_us": round(ws6_2["avg_us"], 3), "bytes_per_launch": int(ws6["bytes_per_launch"])},
            "layer_tables_b1": {"avg_launch_us": round(tables1["avg_launch_us"], 3), "ms_per_pass": round(tables1["ms_per_pass"], 4),
                                "GBs": round(tables1["bytes_per_pass"] / tables1["launches"] / tables1["avg_launch_us"] / 1e3, 1)},
            "layer_tables_b2": {"avg_launch_us": round(tables2["avg_launch_us"], 3), "ms_per_pass": round(tables2["ms_per_pass"], 4)},
            "cfg1_layer_linears": {"workload": "cfg1: one Seoul-shaped layer's linears q 2048x2048, k and v 512x2048, "
                                                   "o 2048x2048, gate and up 8192x2048, down 2048x8192 in Q4_0 through the "
                                                   "kernel-level GEMV (int8 cut per 32 columns), 16 copies in rotation",
                                   "table_bytes": layer_bytes,
                                   "b1_us": round(l_us1, 2), "b2_us": round(l_us2, 2),
                                   "b2_GBs": round(layer_bytes / l_us2 / 1e3, 1),
                                   "b2_frac": round(layer_bytes / l_us2 / 1e3 / HBM_PEAK_GBS, 4),
                                   "grouped": {"launches_per_layer": {"b1": 1, "b2": 2}, "b1_us": round(lg_us1, 2), "b2_us": round(lg_us2, 2),
                                               "b2_GBs": round(layer_bytes / lg_us2 / 1e3, 1),
                                               "b2_frac": round(layer_bytes / lg_us2 / 1e3 / HBM_PEAK_GBS, 4),
                                               "outputs_equal_per_table": bool(l_group_same)}},
            "cfg0_gemv_8192x2048": {"avg_us": round(cfg0_us, 3), "GBs": round(cfg0_bytes / cfg0_us / 1e3, 1),
                                    "frac": round(cfg0_bytes / cfg0_us / 1e3 / HBM_PEAK_GBS, 4),
                                    # the same 640 launches captured in one HIP graph (64 copies in order) and
                                    # replayed back to back
                                    "graph_avg_us": round(cfg0_graph_us, 3),
                                    "graph_GBs": round(cfg0_bytes / cfg0_graph_us / 1e3, 1),
                                    "graph_frac": round(cfg0_bytes / cfg0_graph_us / 1e3 / HBM_PEAK_GBS, 4),
                                    "kernel_us": round(cfg0_kernel_us, 3),
                                    "kernel_GBs": round(cfg0_bytes / cfg0_kernel_us / 1e3, 1),
                                    "kernel_frac": round(cfg0_bytes / cfg0_kernel_us / 1e3 / HBM_PEAK_GBS, 4),
                                    "floor": cfg0_floor},
        },
    }
    _progress("cfg 0 and cfg 1 timed")
    if args.real_steps:
        line["real_seoul_decode"] = real_seoul_decode(args.real_steps, args.warmup)
        _progress("Seoul file shape decode timed")
    if args.prefill_reps:
        pt, plg, pbest = gpu_prefill(brain, args.prefill_reps)
        n_pf = HEAR_EMB + HEAR_TOK
        # integer ops of the layer tables (2 per weight per position) and of the last position's word scores
        layer_weights = (brain.table_bytes - brain.n_vocab * brain.n_embd * 18 // 32) * 32 // 18
        ops = 2 * n_pf * layer_weights + 2 * brain.n_vocab * brain.n_embd
        line["prefill"] = {
            "workload": f"cfg3: hearing window, {HEAR_EMB} fp32 embedding rows ~N(0,1) then {HEAR_TOK} seeded words, one "
                        "causal prefill of the cfg2 model (KV written), last-position word scores",
            "positions": n_pf,
            "best_ms": round(float(pt.min()) * 1e3, 3),
            "p50_ms": round(float(np.percentile(pt, 50)) * 1e3, 3),
            "positions_per_s": round(n_pf / float(np.percentile(pt, 50)), 1),
            "int8_tops": round(ops / float(np.percentile(pt, 50)) / 1e12, 2),
            "int8_peak_tops": 5000.0,
            "mfma_util_pct_counter_run": PREFILL_MFMA_UTIL_PCT,
            "mfma_util_source": "counter run (not this process): profiles/prefill_hearing_window_seoul.md",
            "reps": int(len(pt)),
        }
    _progress("prefill timed")
    if args.hear_reps:
        epath = synth.cached("ears", synth.EARS, 3)
        te, tp, hrows, hlg, hbest, einfo = gpu_hear(brain, epath, args.hear_reps)
        n_fr = (HEAR_SAMPLES - 400 + 159) // 160 + 1
        fma = ears_fma(einfo, HEAR_EMB, n_fr)
        e50 = float(np.percentile(te, 50))
        line["hear"] = {
            "workload": f"the hearing window from sound: {HEAR_SAMPLES / 16000:.2f} s of seeded 16 kHz samples through the "
                        f"ears ({n_fr} mel frames of 128 bands, stride-2 downsampler to {HEAR_EMB} positions, "
                        f"{einfo.n_layer} causal LFM layers ({einfo.n_attn} attention over {einfo.window} positions), "
                        f"{einfo.n_embd} wide, F16 tables, projector to 2048), then the {HEAR_EMB} rows and "
                        f"{HEAR_TOK} seeded words as one causal prefill of the cfg2 model",
            "ears_p50_ms": round(e50 * 1e3, 3),
            "prefill_p50_ms": round(float(np.percentile(tp, 50)) * 1e3, 3),
            "total_p50_ms": round(float(np.percentile(te + tp, 50)) * 1e3, 3),
            "ears_fma": int(fma),
            "ears_tflops": round(2 * fma / e50 / 1e12, 2),
            "fp32_valu_peak_tflops": 78.6,
            "ears_table_bytes": int(einfo.table_bytes),
            "reps": int(len(te)),
        }
    _progress("hearing from sound timed")
    if args.voice_frames:
        vpath = synth.cached("voice", synth.VOICE, 1)
        (ft, fbr, fvo, fcodes, fids, _), fref, vinfo = gpu_voice_frames(path, vpath, args.voice_frames, VOICE_WARMUP)
        # algorithmic bytes of a frame: the step2 (every brain table once, the word table for slot A's scores, the
        # fp32 vectors, and the K and V rows each slot's attention reads at its position), then the generator (its
        # proj_in once, its layer tables once per pass, the 8 score tables of the frame's codebooks once each)
        vs = synth.VOICE
        q8 = lambda rows, cols: (rows + 7) // 8 * 8 * (cols // 32) * 34
        heads_b = vs.n_cb * q8(vs.n_vocab, vs.n_embd)
        proj_b = q8(vs.n_cb * vs.n_embd, vs.n_in)
        layers_b = int(vinfo["table_bytes"]) - heads_b - proj_b
        gen_b = proj_b + len(SCHEDULE) * layers_b + heads_b
        kv_row = brain.n_attn * brain.n_head_kv * brain.head_dim * 2
        nfr = len(ft)
        kv_b = sum(2 * kv_row * ((A_POS + VOICE_WARMUP + f + 1) + (VOICE_WARMUP + f + 1)) for f in range(nfr)) / nfr
        brain_b = brain.table_bytes + brain.vector_bytes + kv_b
        frame_b = brain_b + gen_b
        p50 = float(np.percentile(ft, 50))
        line["voice_frame"] = {
            "workload": "cfg4: step2 of the cfg2 model (slot A: text step with scores at KV context 4096, from position "
                        f"{A_POS}; slot B: voice brain step fed the feedback row sum), then the Q8_0 generator "
                        "(6 layers, hidden 1024, FFN 4096, 16/4 heads x 64, 8 codebooks x 2048) in passes of 4 + 4 "
                        "codebooks in a shuffled order, each followed by sampling on the device (temperature 0.4, "
                        "repeat penalty 1.2 over the last 64 frames), and the feedback row sum",
            "frames": int(len(ft)),
            "p50_ms": round(float(np.percentile(ft, 50)) * 1e3, 3),
            "p99_ms": round(float(np.percentile(ft, 99)) * 1e3, 3),
            "mean_ms": round(float(ft.mean()) * 1e3, 3),
            "step2_p50_ms": round(float(np.percentile(fbr, 50)) * 1e3, 3),
            "generator_p50_ms": round(float(np.percentile(fvo, 50)) * 1e3, 3),
            "generator_table_bytes": int(vinfo["table_bytes"]),
            "bytes_per_frame": {"step2": int(brain_b), "generator": int(gen_b), "total": int(frame_b)},
            "GBs_at_p50": round(frame_b / p50 / 1e9, 1),
            "hbm_frac_at_p50": round(frame_b / p50 / 1e9 / HBM_PEAK_GBS, 4),
            "budget_ms": 80.0,
        }
    _progress("voice frames timed")
    if args.talk_frames:
        tpath = synth.cached("voice", synth.TALK_VOICE, 1)
        cpath = synth.cached("codec", synth.CODEC, 2)
        (tt, tbr, tvo, _, _, tcd), tref, tinfo = gpu_voice_frames(path, tpath, args.talk_frames, 4, PROMPT,
                                                                  TALK_SCHEDULE, cpath)
        line["talk_frame"] = {
            "workload": "a whole talk frame as imi's talk loop runs it at the generator's own shape: step2 of the cfg2 "
                        f"model (slot A from position {PROMPT}), the Q8_0 generator (3 layers, hidden 1024, FFN 4096, "
                        "16/4 heads x 64, 12 codebooks x 2048) in passes of 6 + 6 codebooks with sampling on the "
                        "device, then the codec (12 codes -> FSQ -> 8 LFM layers on Q8_0, 512 wide, 5 short conv + 3 "
                        "gated attention over 30 positions -> 1280-point inverse STFT, 1920 samples at 24 kHz) and "
                        "the feedback row sum",
            "frames": int(len(tt)),
            "p50_ms": round(float(np.percentile(tt, 50)) * 1e3, 3),
            "p99_ms": round(float(np.percentile(tt, 99)) * 1e3, 3),
            "step2_p50_ms": round(float(np.percentile(tbr, 50)) * 1e3, 3),
            "generator_p50_ms": round(float(np.percentile(tvo, 50)) * 1e3, 3),
            "codec_p50_ms": round(float(np.percentile(tcd, 50)) * 1e3, 3),
            "generator_table_bytes": int(tinfo["table_bytes"]),
            "codec_table_bytes": tinfo["codec_table_bytes"],
            "audio_ms_per_frame": 80.0,
        }
    _progress("talk frames timed")
    if not args.no_cpu:
        import oracle
        # the CPU path built for this host (-O3 -march=native; the portable x86-64-v3 build if that fails)
        native = oracle.use_native()
        cpu_build = "-O3 -march=native on this host" if native else "-O3 -march=x86-64-v3 (portable build)"
        _progress(f"CPU path built: {cpu_build}")
        info = cpu_info()
        aff = info["logical_cpus"]
        threads = args.cpu_threads or min(16, aff)
        cpu_steps = min(args.steps, 256)
        runs1, runs2 = args.cpu_runs, max(1, args.cpu_runs // 2)
        c1, cids, csecs = cpu_decode(path, threads, cpu_steps, b2=False, runs=runs1)
        c2, cids2, csecs2 = cpu_decode(path, threads, cpu_steps, b2=True, runs=runs2)
        c4, _, csecs4 = cpu_decode(path, 4, cpu_steps, b2=False, runs=1)   # imi's own setting: 4 threads
        n1, n2 = min(len(cids), len(ids_b1)), min(len(cids2[0]), len(ids_b2[0]))
        same = bool(np.array_equal(cids[:n1], ids_b1[:n1]))
        same2 = bool(np.array_equal(cids2[0][:n2], ids_b2[0][:n2]) and np.array_equal(cids2[1][:n2], ids_b2[1][:n2]))
        line["cpu_baseline"] = {
            "value": round(c1, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"cfg2 B=1: {runs1} conversations of a {PROMPT}-token seeded prompt then {cpu_steps} greedy ids "
                      f"({csecs:.1f} s generating); B=2: {runs2} step2 pairs of {cpu_steps} positions ({csecs2:.1f} s) = "
                      f"{c2:.2f} tokens/s; 4 threads (imi's README setting): one conversation, {c4:.2f} tokens/s "
                      f"({csecs4:.1f} s); {threads} threads of {aff} logical CPUs in the affinity mask "
                      f"({info['physical_cores']} physical cores, SMT width {info['smt_width']}), {info['model']}; "
                      f"oracle/ C++ restatement of imi's AVX2 engine, {cpu_build}, imi's spinning thread team",
            "build": cpu_build,
            "b2_value": round(c2, 2),
            "four_thread_value": round(c4, 2),
            "cpu": info,
        }
        line["speedup_vs_cpu"] = {"b1": round(tok_s_b1 / c1, 1), "b2": round(tok_s_b2 / c2, 1),
                                  "b1_vs_4_threads": round(tok_s_b1 / c4, 1)}
        line["greedy_ids_match_cpu"] = same
        line["greedy_ids_match_cpu_b2"] = same2
        # cfg 0 and cfg 1 on the CPU (imi's q4x8 figure of merit is table GB/s on one thread)
        g1, gt = cpu_cfg0(1), cpu_cfg0(threads)
        line["kernels"]["cfg0_gemv_8192x2048"]["cpu"] = {"GBs_1_thread": round(g1, 2), f"GBs_{threads}_threads": round(gt, 2),
                                                         "kind": "port", "sample": "oracle q4x8 GEMV (imi/kernels/q4x8.cpp) "
                                                         "8192 x 2048, fastest rep of about 2 s of reps on one table"}
        cl1, cl2, cl_out = cpu_layer(threads)
        line["kernels"]["cfg1_layer_linears"]["cpu"] = {
            "b1_us": round(cl1, 1), "b2_us": round(cl2, 1), "cores": threads, "kind": "port",
            "sample": "oracle group / group2 kernels (imi/core/tables.cpp), each table's fastest rep, about 2 s of reps per batch size"}
        line["kernels"]["cfg1_layer_linears"]["speedup_vs_cpu"] = {"b1": round(cl1 / l_us1, 1), "b2": round(cl2 / l_us2, 1),
                                                                   "grouped_b1": round(cl1 / lg_us1, 1),
                                                                   "grouped_b2": round(cl2 / lg_us2, 1)}
        line["kernels"]["cfg1_layer_linears"]["outputs_match_cpu"] = bool(all(
            np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32)) for a, b in zip(l_out, cl_out)))
        if args.prefill_reps:
            csec, clg = cpu_prefill(path, threads)
            line["prefill"]["cpu"] = {"ms": round(csec * 1e3, 1), "cores": threads, "kind": "port",
                                      "sample": "one hearing-window prefill on the oracle (imi's step_batch restated)"}
            line["prefill"]["speedup_vs_cpu"] = round(csec / float(np.percentile(pt, 50)), 1)
            line["prefill"]["scores_match_cpu"] = bool(np.array_equal(clg.view(np.uint32), plg.view(np.uint32)))
        if args.hear_reps:
            ce, cp, crows, clg2 = cpu_hear(path, epath, threads)
            line["hear"]["cpu"] = {"ears_ms": round(ce * 1e3, 1), "prefill_ms": round(cp * 1e3, 1), "cores": threads,
                                   "kind": "port", "sample": "one encode (after one untimed) and one prefill on the oracle "
                                   "(imi's ears and step_batch restated, AVX2, imi's spinning thread team)"}
            line["hear"]["speedup_vs_cpu"] = round((ce + cp) / float(np.percentile(te + tp, 50)), 1)
            line["hear"]["rows_rel_l2_vs_cpu"] = float(oracle_rel(hrows, crows))
            line["hear"]["scores_rel_l2_vs_cpu"] = float(oracle_rel(hlg, clg2))
            line["hear"]["best_id_matches_cpu"] = bool(int(np.argmax(clg2)) == int(hbest))
        if args.voice_frames and args.cpu_voice_frames:
            ct, cbr, cvo, ccodes, cids, _, _, _, _ = cpu_voice_frames(path, vpath, threads, args.cpu_voice_frames)
            n = len(ct)
            line["voice_frame"]["cpu"] = {
                "p50_ms": round(float(np.percentile(ct, 50)) * 1e3, 2),
                "step2_p50_ms": round(float(np.percentile(cbr, 50)) * 1e3, 2),
                "generator_p50_ms": round(float(np.percentile(cvo, 50)) * 1e3, 2),
                "frames": n, "cores": threads, "kind": "port",
                "sample": f"the first {n} frames of the same run on the oracle (C++ restatement of imi's engine and voice "
                          "generator; its 8-codebook pass tables take imi's scalar generic order)",
            }
            line["voice_frame"]["codes_match_cpu"] = bool(np.array_equal(ccodes, fref[3][:n]) and cids == fref[4][:n])
        if args.talk_frames and args.cpu_talk_frames:
            ct, cbr, cvo, ccodes, cids, _, _, ccd, cpcm = cpu_voice_frames(path, tpath, threads, args.cpu_talk_frames,
                                                                           PROMPT, TALK_SCHEDULE, cpath)
            n = len(ct)
            line["talk_frame"]["cpu"] = {
                "p50_ms": round(float(np.percentile(ct, 50)) * 1e3, 2),
                "step2_p50_ms": round(float(np.percentile(cbr, 50)) * 1e3, 2),
                "generator_p50_ms": round(float(np.percentile(cvo, 50)) * 1e3, 2),
                "codec_p50_ms": round(float(np.percentile(ccd, 50)) * 1e3, 2),
                "frames": n, "cores": threads, "codec_cores": 1, "kind": "port",
                "sample": f"the first {n} frames of the same run on the oracle (C++ restatement of imi's engine, voice "
                          "generator with its 12-input AVX2 table order, and codec on one thread)",
            }
            line["talk_frame"]["codes_match_cpu"] = bool(np.array_equal(ccodes, tref[3][:n]) and cids == tref[4][:n])
            gp = tref[8][:len(cpcm)].astype(np.float64)
            line["talk_frame"]["pcm_rel_l2_vs_cpu"] = float(
                np.sqrt(((gp - cpcm) ** 2).sum() / max((cpcm.astype(np.float64) ** 2).sum(), 1e-30)))
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
