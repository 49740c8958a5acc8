"""Decode-attention layer-step benchmark on one MI355X.

A step is one decode step over every layer of the configuration.  Per layer it runs
quantize-on-append of the new token's K/V and split-K quantized decode attention over
the whole context:
both in one launch (kvq_append_decode_attn) of the tiled kernel of the configuration's
format, whose chunk partials are merged in the same launch (at most 64 chunks per KV
head):
- configs 2, 3: INT4-asymmetric K (4 fp16 outlier channels) and TILE32 V;
- config 1: static-scale INT8 K and V in token rows;
- config 4: static-scale INT8 K and TILE32 INT4-asymmetric V.

Caches are seeded synthetic data of the configured shape, one distinct cache per
layer, built on the GPU with the same HIP append kernel.  Each step rewrites the
last slot and attends over the full context, so every step does identical work.
Uniform contexts are passed by value, as the cache engines pass them; the ragged batch of
config 4 passes its per-row lengths (a device tensor), so the kernel shares its
work-groups out over the rows by length.

The timed region runs W warm-up and then K timed steps, bracketed by hipEvents on the
launch stream, both as direct launches and as replays of a HIP graph of one step; the
faster is reported.  ``value`` is the mean microseconds per layer-step (append +
attention).  The line also carries:
- ``roofline``: algorithmic bytes of the dominant kernel (the fused step kernel, else
  the attention kernel) / its measured time per layer;
- ``attention_us_per_layer_step`` / ``append_us_per_layer_step``: each half timed alone
  (its own HIP graph), as a breakdown;
- ``stream_ceiling``: the library's streaming-read probe (kvq_stream_read) over the same
  bytes per launch, replayed from a HIP graph (device time), the read rate this GPU
  sustains for a launch of that size;
- ``engine_api``: the same step through the cache engine a caller uses
  (``cache.append_decode_attn`` per layer, Python included);
- ``int4_fused`` (configuration 3): the reference's ``int4_fused`` kv_mode (group 16,
  outlier rescue 0.01, static tables) through INT4KVCache at the same shape;
- ``cpu_baseline``: the CPU oracle (the reference's torch path restated) timed on a
  bounded sample on this host's cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
MIN_ROTATE = 4  # distinct caches timed in turn for single-layer configurations


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-engine", action="store_true", help="skip the engine-API leg")
    ap.add_argument("--no-modes", action="store_true",
                    help="skip the int4_fused leg (the reference's kv_mode through INT4KVCache "
                         "at configuration 3's shape, reported as the line's int4_fused key)")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the streaming-read ceiling (counter runs)")
    ap.add_argument("--launch", choices=["auto", "graph", "stream"], default="auto",
                    help="how the timed steps are launched: a HIP graph of one step replayed, "
                         "direct launches on the stream, or both timed and the faster reported")
    ap.add_argument("--no-graph", action="store_true", help="same as --launch stream")
    ap.add_argument("--chunk", type=int, default=0)
    ap.add_argument("--layers", type=int, default=0, help="override the layer count (debug only)")
    ap.add_argument("--no-breakdown", action="store_true",
                    help="time only the layer-step (no attention-only / append-only graphs), "
                         "so a profiler sees only the step's launches")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a 1 GiB device copy three times (rocprof counter calibration)")
    ap.add_argument("--kv-mode", choices=sorted(MODE_SETTINGS), default=None,
                    help="time one of the reference's kv_modes through its cache engine at the "
                         "configuration's shape (shipped calibration settings) and exit")
    ap.add_argument("--e2e", default=None, metavar="MODEL",
                    help="end-to-end decode through generate_from_ids on a random-weight "
                         "model of this shape (qwen2.5-1.5b or qwen2.5-7b): TTFT / TPOT per "
                         "kv_mode, one JSON line per mode")
    ap.add_argument("--prompt", type=int, default=4096, help="--e2e prompt length")
    ap.add_argument("--new-tokens", type=int, default=32, help="--e2e generated tokens")
    ap.add_argument("--e2e-modes", default="fp16,int8_ours,int4_fused",
                    help="--e2e kv_modes (comma separated)")
    ap.add_argument("--kivi-probe", action="store_true",
                    help="only time kvq_decode_attn over the KIVI layout at config 3's shape "
                         "(B 8, 28 / 4 heads, 32k tokens; random codes and parameters)")
    return ap.parse_args()


def append_bytes(cfg):
    """Bytes of one layer's quantize-on-append: fp16 K and V rows in, codes (+ fp16
    outlier channels) out, for every (b, kv head)."""
    out = ((128 if cfg.k_format == "int8" else 64) + (128 if cfg.v_format == "int8" else 64)
           + (8 if cfg.outlier_channels else 0))
    return cfg.batch * cfg.kv_heads * (2 * 128 * 2 + out)


def algorithmic_bytes(cfg, ctx_list):
    """Bytes one layer-step must move: codes (+ fp16 outlier channels / per-token
    scales the format stores) for every context token, plus q in and out."""
    tok = sum(int(c) for c in ctx_list)
    per_tok_head = 0
    per_tok_head += 128 if cfg.k_format == "int8" else 64
    per_tok_head += 128 if cfg.v_format == "int8" else 64
    if cfg.outlier_channels:
        per_tok_head += 4 * 2
    return tok * cfg.kv_heads * per_tok_head + 2 * cfg.batch * cfg.q_heads * 128 * 2


class Layer:
    """Device buffers and prepared C-ABI calls of one layer."""

    def __init__(self, cfg, layer, device, ctx, gen, chunk):
        from llm_kvcache_quantization_amd import _capi as C
        from llm_kvcache_quantization_amd import synthetic as SY
        from llm_kvcache_quantization_amd.kernels import DecodePlan, kv_view_static, kv_view_tok

        self.C = C
        B, Hkv, Hq = cfg.batch, cfg.kv_heads, cfg.q_heads
        cap = int(max(ctx))
        if cfg.v_format != "int8":
            cap = -(-cap // 32) * 32  # TILE32 V holds whole 32-token tiles
        t = SY.calibrate(cfg, layer % cfg.layers)
        self.tables = t
        ch = SY.outlier_channels(cfg, layer % cfg.layers)
        kb = 128 if cfg.k_format == "int8" else 64
        vb = 128 if cfg.v_format == "int8" else 64
        self.k = torch.empty(B, Hkv, cap, kb, dtype=torch.uint8, device=device)
        # asymmetric INT4 V in the TILE32 layout (as INT4AsymKVCache keeps it), which the
        # tiled kernels read with INT4-asymmetric or static INT8 K
        self.v_tiled = cfg.v_format != "int8"
        if self.v_tiled:
            assert cap % 32 == 0
            self.v = torch.empty(B, Hkv, cap // 32, 2048, dtype=torch.uint8, device=device)
        else:
            self.v = torch.empty(B, Hkv, cap, vb, dtype=torch.uint8, device=device)
        self.ko = None
        dev = lambda x: None if x is None else x.to(device)
        self.ks, self.kz = dev(t.k_scale), dev(t.k_zp)
        self.vs, self.vz = dev(t.v_scale), dev(t.v_zp)
        self.oidx = dev(t.k_outlier_idx)
        if cfg.outlier_channels:
            self.ko = torch.empty(B, Hkv, cap, 4, dtype=torch.float16, device=device)
        self.ctx = torch.tensor(ctx, dtype=torch.int32, device=device)
        self.q = SY.draw_q(cfg, B, gen, device=device)
        self.inv_tau = SY.inv_tau(cfg)[layer % cfg.layers].to(device)
        # prefill: every slot [0, cap) gets quantized seeded data (chunks bound the temporaries)
        step = 8192
        for s0 in range(0, cap, step):
            n = min(step, cap - s0)
            kx, vx = SY.draw_kv(cfg, layer % cfg.layers, B, n, gen, device=device, ch=ch)
            pk, pv = self._append_params(cfg, kx, vx, s0)
            C.check(C.lib().kvq_quant_append(ctypes.byref(pk), ctypes.byref(pv),
                                             ctypes.c_void_p(C.stream_handle(torch.device(device)))))
            del kx, vx
        # the decode-step token: rewrites slot cap-1 of every sequence each step
        self.k_new, self.v_new = SY.draw_kv(cfg, layer % cfg.layers, B, 1, gen, device=device, ch=ch)
        self.step_slot = cap - 1
        self.pk, self.pv = self._append_params(cfg, self.k_new, self.v_new, self.step_slot)
        self._pk, self._pv = ctypes.byref(self.pk), ctypes.byref(self.pv)
        ks_view = None
        if cfg.k_format == "int8":
            self.ks_tok = self.ks.clamp(min=1e-5).to(torch.float16)[None, :, None, :].expand(B, Hkv, cap, 4)
            kview = kv_view_tok(self.k, self.ks_tok)
            kfmt = C.KVQ_FMT_INT8_SYM
        else:
            kview = kv_view_static(self.k, self.ks, self.kz, self.oidx, self.ko)
            kfmt = C.KVQ_FMT_INT4_ASYM
        if cfg.v_format == "int8":
            self.vs_tok = self.vs.clamp(min=1e-5).to(torch.float16)[None, :, None, :].expand(B, Hkv, cap, 4)
            vview = kv_view_tok(self.v, self.vs_tok)
            vfmt = C.KVQ_FMT_INT8_SYM
        else:
            vview = kv_view_static(self.v, self.vs, self.vz)
            vfmt = C.KVQ_FMT_INT4_ASYM
        del ks_view
        # uniform contexts go by value, as the cache engines pass them (every row has the
        # same length); a ragged batch passes its per-row lengths
        ctx_arg = int(ctx[0]) if cfg.ragged_min is None else self.ctx
        self.plan = DecodePlan(self.q, kfmt, kview, vfmt, vview, ctx_arg, Hkv, cap,
                               1.0 / math.sqrt(128), 32, inv_tau=self.inv_tau, chunk_tokens=chunk)
        # every configuration's format has a tiled kernel, so kvq_append_decode_attn does
        # the step (append + attention) in one launch
        self.fused = True

    def _append_params(self, cfg, kx, vx, pos):
        C = self.C
        out = []
        for x, codes, fmt, s, z, side in ((kx, self.k, cfg.k_format, self.ks, self.kz, "k"),
                                          (vx, self.v, cfg.v_format, self.vs, self.vz, "v")):
            p = C.AppendParams()
            B, H, S, D = x.shape
            p.format = C.KVQ_FMT_INT8_SYM if fmt == "int8" else C.KVQ_FMT_INT4_ASYM
            p.x = x.data_ptr()
            p.x_stride_b, p.x_stride_h, p.x_stride_s = x.stride(0), x.stride(1), x.stride(2)
            p.batch, p.heads, p.seq_new, p.head_dim, p.group_size = B, H, S, D, 32
            p.static_scale = s.data_ptr()
            p.static_scale_dtype = C.KVQ_DTYPE_F16
            p.static_stride_h, p.static_stride_g = s.stride()
            if z is not None:
                p.static_zp = z.data_ptr()
            p.codes = codes.data_ptr()
            p.codes_stride_b, p.codes_stride_h, p.codes_stride_t = codes.stride(0), codes.stride(1), codes.stride(2)
            p.write_pos = pos
            p.capacity = codes.shape[2]
            if side == "v" and self.v_tiled:
                p.codes_layout = C.KVQ_LAYOUT_TILE32
                p.codes_stride_t = 64
                p.capacity = codes.shape[2] * 32
            if side == "k" and self.ko is not None:
                p.n_outlier = 4
                p.outlier_idx = self.oidx.data_ptr()
                p.outlier_out = self.ko.data_ptr()
                p.oo_stride_b, p.oo_stride_h, p.oo_stride_t = self.ko.stride(0), self.ko.stride(1), self.ko.stride(2)
            p._keep = (x,)
            out.append(p)
        return out

    def append(self, stream):
        self.C.check(self.C.lib().kvq_quant_append(self._pk, self._pv, ctypes.c_void_p(stream)))

    def attend(self, stream):
        self.plan.launch(stream)

    def step(self, stream):
        """One decode layer-step: one fused launch (append + attention) where the format
        has it, else the append launch then the attention launch."""
        if self.fused:
            self.plan.launch_append(self.pk, self.pv, stream)
        else:
            self.append(stream)
            self.attend(stream)


def time_region(fn, stream, steps, warmup, use_graph):
    """Mean ms per call of fn(stream) over `steps` calls, timed with HIP events."""
    s = torch.cuda.current_stream()
    for _ in range(2):
        fn(s.cuda_stream)
    torch.cuda.synchronize()
    graph = None
    if use_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn(torch.cuda.current_stream().cuda_stream)
        run = graph.replay
    else:
        run = lambda: fn(s.cuda_stream)
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, graph


def stream_ceiling(device, nbytes, reps=28):
    """HBM read ceilings of this GPU from kvq_stream_read, the library's streaming-read probe
    (non-temporal 16-byte loads, as the decode kernels read cache codes, XOR-folded):
    - ``read_GBps_same_bytes``: launches of `nbytes` each (the bytes of one decode launch),
      each reading the next window of a 4 GiB buffer, so that, as in the decode step, no
      launch is served from the 256 MB MALL;
    - ``read_GBps_4GiB``: one launch over the whole buffer.
    Each is the best over 1 to 64 work-groups (512 threads, one contiguous slab each) per CU.
    The same-bytes launches are replayed from a HIP graph of `reps` launches, so that the
    figure is device time: from Python, launches of a few MB are host-bound (about 10 us per
    ctypes call)."""
    from llm_kvcache_quantization_amd import _capi as C

    L = C.lib()
    big = 4 << 30
    buf = torch.randint(-2 ** 31, 2 ** 31 - 1, (big // 4,), dtype=torch.int32, device=device)
    nwin = (int(nbytes) // 256) * 256
    nwins = big // nwin
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    s = torch.cuda.current_stream().cuda_stream
    out = {"kernel": "kvq_stream_read", "bytes_per_launch": nwin}
    best_same, best_big = (0.0, 0), (0.0, 0)
    for per_cu in (1, 4, 16, 32, 64):
        wgs = per_cu * cus
        sink = torch.zeros(wgs, dtype=torch.int32, device=device)

        def launch(off, n, stream=s):
            C.check(L.kvq_stream_read(ctypes.c_void_p(buf.data_ptr() + off), n,
                                      ctypes.c_void_p(sink.data_ptr()), wgs,
                                      ctypes.c_void_p(stream)))

        for w in range(nwins):
            launch(w * nwin, nwin)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            cs = torch.cuda.current_stream().cuda_stream
            for r in range(reps):
                launch((r % nwins) * nwin, nwin, cs)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        gbps = nwin * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9
        del graph
        best_same = max(best_same, (gbps, wgs))
        e0.record()
        for _ in range(3):
            launch(0, big)
        e1.record()
        torch.cuda.synchronize()
        gbps = big * 3 / (e0.elapsed_time(e1) * 1e-3) / 1e9
        best_big = max(best_big, (gbps, wgs))
        del sink
    del buf
    out["read_GBps_same_bytes"] = round(best_same[0], 1)
    out["work_groups_same_bytes"] = best_same[1]
    out["us_per_launch_same_bytes"] = round(nwin / (best_same[0] * 1e3), 3)
    out["read_GBps_4GiB"] = round(best_big[0], 1)
    out["work_groups_4GiB"] = best_big[1]
    return out


def engine_leg(cfg, device, steps, warmup):
    """The engine API a caller uses: ``cache.append_decode_attn(layer, q, k, v, sm_scale,
    inv_tau)`` for every layer of the configuration (a single-layer configuration rotates
    MIN_ROTATE layers, as the main timing does), on the cache engine of its format
    (INT4AsymKVCache, or INT8KVCache with the static group-32 tables), prefilled with
    seeded data through ``append`` to a context a few tokens short of the configuration's,
    so that the timed steps end at it.  Timed with hipEvents as the main loop, with
    check_numerics off (no host read-back) and on (one status read-back per call, as the
    reference's NaN / clip checks synchronise).  None for ragged batches: an engine holds
    one length for all rows."""
    if cfg.ragged_min is not None or cfg.k_format != cfg.v_format:
        return None
    import llm_kvcache_quantization_amd as K
    from llm_kvcache_quantization_amd import synthetic as SY

    nl = max(cfg.layers, MIN_ROTATE)
    calls = 2 + 2 * (warmup + steps)
    s0 = ((cfg.context - calls) // 32) * 32
    tabs = [SY.calibrate(cfg, l % cfg.layers) for l in range(nl)]
    stack = lambda name: torch.stack([getattr(t, name) for t in tabs]).to(device)
    tau = SY.inv_tau(cfg).to(device)
    if cfg.k_format == "int8":
        cache = K.INT8KVCache(nl, device=device, group_size=32, max_seq_len=cfg.context,
                              static_k_scale=stack("k_scale"), static_v_scale=stack("v_scale"),
                              check_numerics=False)
    else:
        cache = K.INT4AsymKVCache(nl, stack("k_scale"), stack("k_zp"), stack("v_scale"), stack("v_zp"),
                                  device=device, max_seq_len=cfg.context,
                                  k_outlier_idx=stack("k_outlier_idx") if cfg.outlier_channels else None)
    gen = torch.Generator(device=device).manual_seed(SY.seed_for(cfg.index, 0) + 5)
    for l in range(nl):
        k, v = SY.draw_kv(cfg, l % cfg.layers, cfg.batch, s0, gen, device=device)
        cache.append(l, k, v)
        del k, v
    q = SY.draw_q(cfg, cfg.batch, gen, device=device)
    k1, v1 = SY.draw_kv(cfg, 0, cfg.batch, 1, gen, device=device)
    sm = 1.0 / math.sqrt(128)
    taus = [tau[l % cfg.layers].contiguous() for l in range(nl)]

    def step():
        for l in range(nl):
            cache.append_decode_attn(l, q, k1, v1, sm, inv_tau=taus[l])

    step()          # the first call grows each layer's buffer to the full context
    torch.cuda.synchronize()
    res = {"engine": type(cache).__name__, "layers": nl}
    for checked in (False, True):
        cache.check_numerics = checked
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        host = time.perf_counter() - t0
        torch.cuda.synchronize()
        key = "checked" if checked else "unchecked"
        res[f"us_per_layer_step_{key}"] = round(e0.elapsed_time(e1) * 1e3 / (steps * nl), 3)
        res[f"host_us_per_call_{key}"] = round(host * 1e6 / (steps * nl), 3)
    res["context_timed"] = [s0 + 2 + warmup, cache.get_seq_len()]
    cache.release()
    return res


# The reference's own kv_modes with the settings its shipped calibration files carry
# (artifacts/kv_calib_mse_1p5b_int8.json / _int4.json: group 16, int4_outlier_ratio 0.01;
# loaded by src/engine/generate_loop.py:751-889): static tables for the *_ours / *_fused
# modes, dynamic per-token scales for the baselines.
MODE_SETTINGS = {
    "int8_baseline": dict(static=False, group_size=128),
    "int8_fused": dict(static=False, group_size=128),
    "int8_ours": dict(static=True, group_size=16),
    "int4_baseline": dict(static=False, group_size=32),
    "int4_fused": dict(static=True, group_size=16, outlier_rescue_ratio=0.01),
    "int4_ours": dict(static=True, group_size=16, outlier_rescue_ratio=0.01),
    "int4_ours_mixed": dict(static=True, group_size=16, outlier_rescue_ratio=0.01, mixed_rescue=True),
    # KIVI family and the mixed cache (per-channel K frozen at prefill, per-token V; the
    # mixed cache's dynamic INT8 K in groups of 128 with per-token asymmetric INT4 V)
    "kivi_style": dict(family=True, group_size=128),
    "int4_kivi_aligned": dict(family=True, group_size=128),
    "int4_mixed_kv": dict(family=True, group_size=128),
}


def modes_leg(cfg, mode, device, steps, warmup):
    """One of the reference's kv_modes at configuration cfg's model shape, batch and
    context: the engine modes.create_kv_cache builds for it, with static tables (when the
    mode has them) from the configuration's seeded calibration sample at the shipped
    settings (MODE_SETTINGS), and per-head inverse temperatures.  Each layer is prefilled
    through ``append`` a few tokens short of the context; then ``append_decode_attn`` runs
    for every layer per step (check_numerics off: no host read-back), timed with
    hipEvents.  Algorithmic bytes per call: each context token's K and V codes and the
    per-token scales (and zero-points) the engine stores (static tables: none), the KIVI
    family's per-channel K parameters once per (b, kv head), q and out."""
    import llm_kvcache_quantization_amd as K
    from llm_kvcache_quantization_amd import calib as CB
    from llm_kvcache_quantization_amd import modes as M
    from llm_kvcache_quantization_amd import synthetic as SY

    if cfg.ragged_min is not None:
        raise SystemExit("--kv-mode: an engine holds one context length for all rows; "
                         "use a configuration with uniform contexts (1, 2 or 3)")
    st = MODE_SETTINGS[mode]
    gs = st["group_size"]
    nl = max(cfg.layers, MIN_ROTATE)
    cal = M.Calibration(group_size=gs, clip_percentile=99.9,
                        outlier_rescue_ratio=st.get("outlier_rescue_ratio", 0.0),
                        mixed_rescue=st.get("mixed_rescue", False))
    if st.get("static"):
        make = CB.int8_static_scale if mode.startswith("int8") else CB.int4_static_scale
        ks, vs = [], []
        for l in range(nl):
            g = torch.Generator().manual_seed(SY.seed_for(cfg.index, l % cfg.layers) + 500_000)
            k, v = SY.draw_kv(cfg, l % cfg.layers, 1, SY.CALIB_TOKENS, g)
            ks.append(make(k, gs))
            vs.append(make(v, gs))
        cal.static_k_scale = torch.stack(ks).to(device)
        cal.static_v_scale = torch.stack(vs).to(device)
        cal.inv_tau = SY.inv_tau(cfg).float().to(device)
    calls = 2 + warmup + steps
    s0 = ((cfg.context - calls) // 32) * 32
    family = st.get("family", False)
    if family:
        cache = M.create_kv_cache(mode, nl, device=device, max_seq_len=cfg.context, group_size=gs,
                                  check_numerics=False)
    else:
        cache = M.create_kv_cache(mode, nl, device=device, max_seq_len=cfg.context, calib=cal,
                                  check_numerics=False)
    gen = torch.Generator(device=device).manual_seed(SY.seed_for(cfg.index, 0) + 6)
    for l in range(nl):
        k, v = SY.draw_kv(cfg, l % cfg.layers, cfg.batch, s0, gen, device=device)
        cache.append(l, k, v)
        del k, v
    q = SY.draw_q(cfg, cfg.batch, gen, device=device)
    k1, v1 = SY.draw_kv(cfg, 0, cfg.batch, 1, gen, device=device)
    sm = 1.0 / math.sqrt(128)
    taus = [None if cal.inv_tau is None else cal.inv_tau[l].half().contiguous() for l in range(nl)]

    def step():
        for l in range(nl):
            cache.append_decode_attn(l, q, k1, v1, sm, inv_tau=taus[l])

    step()
    torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    host = time.perf_counter() - t0
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (steps * nl)
    n_mid = s0 + 1 + warmup + (steps + 1) // 2
    per_bh = 0  # bytes read once per (b, kv head): the KIVI family's per-channel K parameters
    if family:
        # every stored tensor: per token ([B, H, n, ...] or [B, H, n]) or per (b, kv head)
        ts = cache.get_kivi_tensors(0) if hasattr(cache, "get_kivi_tensors") else cache.get_mixed_tensors(0)
        n_now = ts[0].shape[2]
        per_tok = 0
        for t in ts:
            if t is None:
                continue
            if t.shape[2] == n_now:
                per_tok += (t.shape[3] if t.ndim == 4 else 1) * t.element_size()
            else:
                per_bh += t[0, 0].numel() * t.element_size()
        fused = getattr(cache, "residual_length", 0) == 0
        tok_scales = None
    else:
        kc, vc, kst, vst = cache._raw_views(0)
        per_tok = kc.shape[-1] + vc.shape[-1]
        for tok, s in ((cache._k_tok[0], kst), (cache._v_tok[0], vst)):
            if tok:
                per_tok += s.shape[-1] * s.element_size()
        fused = cache._fused_step_ok(128, cfg.batch, cfg.kv_heads)
        tok_scales = [bool(cache._k_tok[0]), bool(cache._v_tok[0])]
    nbytes = (cfg.batch * cfg.kv_heads * (n_mid * per_tok + per_bh) +
              2 * cfg.batch * cfg.q_heads * 128 * 2)
    res = {"kv_mode": mode, "engine": type(cache).__name__, "group_size": gs,
           "static_scales": bool(st.get("static")), "per_token_scales": tok_scales,
           "fused_step": bool(fused), "layers": nl, "batch": cfg.batch, "context_mid": n_mid,
           "us_per_layer_step": round(us, 3), "host_us_per_call": round(host * 1e6 / (steps * nl), 3),
           "bytes_per_call": nbytes, "GBps": round(nbytes / us / 1e3, 1),
           "frac_of_8TBps": round(nbytes / us / 8e6, 4)}
    cache.release()
    return res


def copy_probe(device, nbytes=1 << 30, reps=3):
    """A plain copy of known size, for scaling the FETCH_SIZE / WRITE_SIZE counters: each
    launch reads and writes exactly `nbytes`."""
    a = torch.empty(nbytes // 4, dtype=torch.float32, device=device).uniform_()
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": nbytes, "copy_probe_bytes_written": nbytes,
                      "launches": reps}), flush=True)


def kivi_probe(device, steps, warmup):
    """Decode attention over the KIVI layout (packed rows, per-channel K and per-token V fp32
    parameters) at config 3's per-layer shape.  Algorithmic bytes per call: 136 per (token,
    kv head) (64 + 64 code bytes, 8 bytes of V parameters), 1 KiB of K parameters per
    (b, kv head), q read and output written."""
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd import kernels as KK

    B, Hq, Hkv, S = 8, 28, 4, 32768
    g = torch.Generator(device=device).manual_seed(0)
    q = torch.randn(B, Hq, 128, device=device, generator=g).half()
    kp = torch.randint(-128, 127, (B, Hkv, S, 64), device=device, dtype=torch.int8, generator=g)
    vp = torch.randint(-128, 127, (B, Hkv, S, 64), device=device, dtype=torch.int8, generator=g)
    ks = torch.rand(B, Hkv, 128, device=device, generator=g) * 0.2 + 0.01
    kz = torch.randn(B, Hkv, 128, device=device, generator=g)
    vs = torch.rand(B, Hkv, S, device=device, generator=g) * 0.2 + 0.01
    vz = torch.randn(B, Hkv, S, device=device, generator=g)
    ctx = torch.full((B,), S, dtype=torch.int32, device=device)
    plan = KK.DecodePlan(q, C.KVQ_FMT_INT4_KIVI, KK.kv_view_kivi(kp, ks, kz, True),
                         C.KVQ_FMT_INT4_KIVI, KK.kv_view_kivi(vp, vs, vz, False), ctx, Hkv, S,
                         1 / math.sqrt(128), 32)
    for _ in range(warmup):
        plan.launch()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        plan.launch()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    nbytes = B * Hkv * S * 136 + B * Hkv * 128 * 8 + B * Hq * 128 * 4
    print(json.dumps({"kivi_probe_us_per_call": round(us, 3), "bytes_per_call": nbytes,
                      "GBps": round(nbytes / us / 1e3, 1), "frac_of_8TBps": round(nbytes / us / 8e6, 4),
                      "chunk_tokens": plan.chunk_tokens, "steps": steps}), flush=True)


def attention_kernels(cfg, layer):
    """Kernels one kvq_decode_attn call launches for this configuration: the tiled kernels
    (TILE32 V, or static-scale INT8 K) merge their chunk partials themselves when they run
    at most 64 chunks per (b, kv head); otherwise a combine launch follows."""
    p = layer.plan.params
    n_chunks = -(-int(p.capacity) // int(layer.plan.chunk_tokens))
    tiled = layer.v_tiled or cfg.k_format == "int8"  # static-scale INT8 K: tiled family too
    if tiled and n_chunks <= 64:
        return "decode_tiled_kernel (single launch, merge in the last work-group)"
    return ("decode_tiled_kernel" if tiled else "decode_splitk_kernel") + " + combine_kernel"


def measured_traffic(cfg_index):
    """HBM bytes per attention call measured by rocprofv3 counters for this configuration,
    from profiles/traffic.json (FETCH_SIZE and WRITE_SIZE per dispatch, each scaled by the
    factor a copy of known size gives); None if no measurement is recorded."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(f"config{cfg_index}")
    except (OSError, ValueError):
        return None
    return None if rec is None else int(rec["traffic_bytes_per_call"])


def cpu_baseline(cfg, layers_dev):
    """The CPU oracle (reference torch path) on a bounded sample of the workload: one
    whole layer-step of layer 0 (every batch row at the full context): quantize-on-append
    of the new token + fp16-dequant fp32 attention, median of at least 3 runs."""
    from oracle import attn as OA
    from oracle import quant as OQ

    torch.set_num_threads(os.cpu_count() or 1)
    L0 = layers_dev[0]
    rows = cfg.batch
    sl = slice(0, rows)
    t = L0.tables
    ctx = L0.ctx[sl].cpu()
    q = L0.q[sl].cpu()
    tau = L0.inv_tau.cpu()
    k_new, v_new = L0.k_new[sl].cpu(), L0.v_new[sl].cpu()
    if cfg.k_format == "int8":
        kc = L0.k[sl].cpu().view(torch.int8)
        ks = L0.ks_tok[sl].cpu()
    else:
        kc = L0.k[sl].cpu()
        ko = L0.ko[sl].cpu() if L0.ko is not None else None
    if L0.v_tiled:  # the oracle reads packed rows; converted before timing
        from llm_kvcache_quantization_amd.kernels import untile_v
        vc = untile_v(L0.v[sl], L0.k.shape[2]).cpu()
    else:
        vc = L0.v[sl].cpu() if cfg.v_format != "int8" else L0.v[sl].cpu().view(torch.int8)

    def one():
        if cfg.k_format == "int8":
            OQ.quantize_symmetric_int8_with_scale(k_new, t.k_scale, 32)
        else:
            OQ.quantize_asymmetric_static(k_new, t.k_scale, t.k_zp)
        if cfg.v_format == "int8":
            OQ.quantize_symmetric_int8_with_scale(v_new, t.v_scale, 32)
            return OA.decode_attn_int8_torch_ref(OA.prescale_q(q, tau), kc, vc, ks, L0.vs_tok[sl].cpu(),
                                                 ctx, 1 / math.sqrt(128))
        OQ.quantize_asymmetric_static(v_new, t.v_scale, t.v_zp)
        if cfg.k_format == "int8":
            return OA.decode_attn_k8v4_ref(q, kc, ks, vc, t.v_scale, t.v_zp, ctx, 1 / math.sqrt(128), inv_tau=tau)
        return OA.decode_attn_asym_ref(q, kc, vc, t.k_scale, t.k_zp, t.v_scale, t.v_zp, ctx,
                                       1 / math.sqrt(128), inv_tau=tau, k_outlier_idx=t.k_outlier_idx,
                                       k_outlier_val=ko)

    one()  # warm-up
    times = []
    budget = 20.0
    t_start = time.perf_counter()
    while len(times) < 10 and (time.perf_counter() - t_start) < budget or len(times) < 3:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    times.sort()
    med = times[len(times) // 2]
    us_per_layer_step = med * 1e6 * (cfg.batch / rows)
    return {
        "value": round(us_per_layer_step, 1),
        "unit": "us/layer-step",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"oracle (reference torch path restated: quantize-on-append, fp16 dequant, "
                   f"fp32 softmax attention) over {rows} of {cfg.batch} batch rows of layer 0 at "
                   f"full context, median of {len(times)} runs"
                   + (f", scaled x{cfg.batch / rows:g} to the full layer-step" if rows != cfg.batch else "")
                   + f"; os.cpu_count()={os.cpu_count()}"),
    }


# Qwen2.5 decoder shapes for the end-to-end leg (the models' published configurations)
E2E_MODELS = {
    "qwen2.5-1.5b": dict(hidden_size=1536, intermediate_size=8960, num_hidden_layers=28,
                         num_attention_heads=12, num_key_value_heads=2, vocab_size=151936,
                         tie_word_embeddings=True),
    "qwen2.5-7b": dict(hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                       num_attention_heads=28, num_key_value_heads=4, vocab_size=152064,
                       tie_word_embeddings=False),
}
# the shipped calibration settings of the reference's tables
# (artifacts/kv_calib_mse_1p5b_int8.json / _int4.json): group 16, K clip percentile 99.5,
# INT4 group rescue ratio 0.01
E2E_CALIB = dict(group_size=16, clip_percentile=99.5, outlier_ratio=0.01)


def e2e_leg(model_name, prompt, new_tokens, modes, device="cuda:0"):
    """End-to-end greedy decode through ``modes.generate_from_ids`` (prefill through the
    model, then one token per step through the attention hook; the reference's TTFT / TPOT
    protocol, src/engine/generate_loop.py:1320-1529: a device synchronisation around every
    step) on a randomly initialised fp16 Qwen2 model of the named shape, batch 1, random
    prompt ids, ``stop_on_eos=False``.  The int8_ours / int4_fused tables come from the
    model's own prefill K/V over 4 calibration prompts of 512 tokens
    (calib.scales_from_absmax_samples at the shipped settings), with per-head inverse
    temperatures drawn in [0.8, 1.2].  Returns one dict per mode."""
    import tempfile

    from transformers import Qwen2Config, Qwen2ForCausalLM

    from llm_kvcache_quantization_amd import calib as CB
    from llm_kvcache_quantization_amd import modes as M
    from llm_kvcache_quantization_amd.modes import _past_layers

    shape = E2E_MODELS[model_name]
    cfg = Qwen2Config(**shape, max_position_embeddings=max(prompt + new_tokens + 64, 32768),
                      rope_theta=1000000.0, rms_norm_eps=1e-6)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(1234)
    t0 = time.time()
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.float16)
    try:
        with torch.device(device):
            model = Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(prev)
    model.eval()
    print(f"[e2e] {model_name}: random fp16 weights in {time.time() - t0:.1f}s", file=sys.stderr,
          flush=True)
    L, Hq = shape["num_hidden_layers"], shape["num_attention_heads"]
    gen = torch.Generator(device=device).manual_seed(4321)
    vocab = shape["vocab_size"]
    # calibration samples: the model's own K / V
    ks_samples, vs_samples = [], []
    with torch.no_grad():
        for _ in range(4):
            ids = torch.randint(0, vocab, (1, 512), device=device, generator=gen)
            pkv = model(input_ids=ids, use_cache=True).past_key_values
            layers = _past_layers(pkv)
            ks_samples.append([k[0].float() for k, _ in layers])
            vs_samples.append([v[0].float() for _, v in layers])
    gs = E2E_CALIB["group_size"]
    ab_k = CB.collect_absmax_samples(ks_samples, gs)
    ab_v = CB.collect_absmax_samples(vs_samples, gs)
    tau = torch.empty(L, Hq).uniform_(0.8, 1.2, generator=torch.Generator().manual_seed(7))
    tmp = tempfile.mkdtemp(prefix="kvq_e2e_")
    files = {}
    for bits, qmax in ((8, 127), (4, 7)):
        d = CB.calibration_json(CB.scales_from_absmax_samples(ab_k, E2E_CALIB["clip_percentile"], qmax),
                                CB.scales_from_absmax_samples(ab_v, E2E_CALIB["clip_percentile"], qmax),
                                group_size=gs, clip_percentile_k=E2E_CALIB["clip_percentile"],
                                inv_tau=tau, quant_bits=bits,
                                outlier_ratio=E2E_CALIB["outlier_ratio"])
        files[bits] = os.path.join(tmp, f"calib_int{bits}.json")
        with open(files[bits], "w") as f:
            json.dump(d, f)
    ids = torch.randint(0, vocab, (1, prompt), device=device, generator=gen)
    out = []
    for mode in modes:
        calib_file = files[4] if mode.startswith("int4") else files[8] if mode.startswith("int8") else None
        kw = dict(kv_mode=mode, calib_file=calib_file, stop_on_eos=False,
                  decode_attn_impl="triton_fused")
        # untimed warm-up (kernels, allocator), then the measured generation
        M.generate_from_ids(model, None, ids[:, :256], max_new_tokens=4, **kw)
        r = M.generate_from_ids(model, None, ids, max_new_tokens=new_tokens, **kw)
        dts = sorted(r.decode_times_ms)
        line = {
            "metric": "end-to-end TTFT / TPOT (generate_from_ids)",
            "model": f"{model_name} (random fp16 weights)", "kv_mode": mode,
            "batch": 1, "prompt": prompt, "new_tokens": new_tokens,
            "ttft_ms": round(r.ttft_ms, 3), "tpot_ms": round(r.tpot_ms, 3),
            "tpot_median_ms": round(dts[len(dts) // 2], 3) if dts else None,
            "kv_cache_mb": round(r.kv_cache_mem_mb, 1),
            "decode_attn_impl": r.decode_attn_impl,
            "fused_decode_calls": (r.decode_stats or {}).get("fused_decode_calls"),
            "check_numerics": True,
        }
        print(f"[e2e] {line}", file=sys.stderr, flush=True)
        out.append(line)
    return out


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the decode path is "
                          "measured on one MI355X (across GPUs it would shard by KV heads "
                          "and batch rows, each GPU running this kernel on its share)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.copy_probe:
        copy_probe("cuda:0")
        return
    if args.kivi_probe:
        kivi_probe("cuda:0", max(args.steps, 200), max(args.warmup, 20))
        return
    if args.e2e:
        from llm_kvcache_quantization_amd import _capi as C

        C.lib()
        torch.cuda.set_device(0)
        for line in e2e_leg(args.e2e, args.prompt, args.new_tokens,
                            [m for m in args.e2e_modes.split(",") if m]):
            print(json.dumps(line), flush=True)
        return
    if args.kv_mode:
        from llm_kvcache_quantization_amd import _capi as C
        from llm_kvcache_quantization_amd import synthetic as SY

        C.lib()
        torch.cuda.set_device(0)
        print(json.dumps(modes_leg(SY.CONFIGS[args.config], args.kv_mode, "cuda:0", args.steps,
                                   args.warmup)), flush=True)
        return
    from llm_kvcache_quantization_amd import _capi as C
    from llm_kvcache_quantization_amd import synthetic as SY

    C.lib()
    cfg = SY.CONFIGS[args.config]
    nl = args.layers or cfg.layers
    # A single-layer configuration is timed over MIN_ROTATE distinct copies of the layer's
    # cache (seeded like layers 0, 1, ...), so that no step is served from the 256 MB
    # Infinity Cache; the result is still per layer-step.
    if not args.layers and nl < MIN_ROTATE:
        nl = MIN_ROTATE
    device = "cuda:0"
    torch.cuda.set_device(0)
    ctx = SY.context_lengths(cfg).tolist()
    gen = torch.Generator(device=device).manual_seed(SY.seed_for(cfg.index, 0))
    print(f"[bench] building {nl} layer caches for config {cfg.index} ({cfg.name})", file=sys.stderr, flush=True)
    t0 = time.time()
    layers = [Layer(cfg, l, device, ctx, gen, args.chunk) for l in range(nl)]
    torch.cuda.synchronize()
    print(f"[bench] caches ready in {time.time() - t0:.1f}s; chunk={layers[0].plan.chunk_tokens}",
          file=sys.stderr, flush=True)

    launch = "stream" if args.no_graph else args.launch
    step_fn = lambda s: [L.step(s) for L in layers]
    # bring the GPU to its steady state before any timed region (untimed, not counted in
    # --warmup): the first region timed otherwise runs about 2% slow
    s0 = torch.cuda.current_stream().cuda_stream
    t_warm = time.time()
    while time.time() - t_warm < 0.3:
        step_fn(s0)
        torch.cuda.synchronize()
    attn_fn = lambda s: [L.attend(s) for L in layers]
    app_fn = lambda s: [L.append(s) for L in layers]
    # Both ways of launching the same kernels are timed (auto): on this ROCm a graph
    # replay adds about 1 us per kernel over direct launches, which the host keeps ahead
    # of the GPU at this size.  The faster is reported and named in config.launch.
    ms_by = {}
    if launch in ("auto", "stream"):
        ms_by["stream"], _ = time_region(step_fn, None, args.steps, args.warmup, False)
    if launch in ("auto", "graph"):
        ms_by["graph"], _ = time_region(step_fn, None, args.steps, args.warmup, True)
    used = min(ms_by, key=ms_by.get)
    ms_step = ms_by[used]
    use_graph = used == "graph"
    us_attn = us_app = None
    if not args.no_breakdown:
        ms_attn, _ = time_region(attn_fn, None, args.steps, args.warmup, use_graph)
        ms_app, _ = time_region(app_fn, None, args.steps, args.warmup, use_graph)
        us_attn = ms_attn * 1000.0 / nl
        us_app = ms_app * 1000.0 / nl
    us_layer = ms_step * 1000.0 / nl
    nbytes = algorithmic_bytes(cfg, ctx)
    fused = layers[0].fused
    # the dominant kernel: the fused step kernel (append + attention, one launch per layer)
    # where the format has it, else the attention kernel; its algorithmic bytes include the
    # append's (the new rows in, their codes out)
    roof_bytes = nbytes + (append_bytes(cfg) if fused else 0)
    roof_us = us_layer if (fused or us_attn is None) else us_attn
    achieved = roof_bytes / (roof_us * 1e-6) / 1e9
    print(f"[bench] step ms by launch mode {ms_by}; reported: {used}", file=sys.stderr, flush=True)
    print(f"[bench] step {ms_step:.3f} ms = {us_layer:.2f} us/layer-step (fused={fused}; "
          f"attention alone {us_attn} us, append alone {us_app} us); {achieved:.0f} GB/s",
          file=sys.stderr, flush=True)

    ceiling = None if args.no_ceiling else stream_ceiling(device, roof_bytes)
    print(f"[bench] stream ceiling {ceiling}", file=sys.stderr, flush=True)
    eng = None
    if not args.no_engine:
        print("[bench] timing the engine API", file=sys.stderr, flush=True)
        eng = engine_leg(cfg, device, args.steps, args.warmup)
        print(f"[bench] engine API {eng}", file=sys.stderr, flush=True)
    fused_mode = None
    if not args.no_modes and cfg.index == 3:
        print("[bench] timing the int4_fused kv_mode at this shape", file=sys.stderr, flush=True)
        fused_mode = modes_leg(cfg, "int4_fused", device, args.steps, args.warmup)
        print(f"[bench] int4_fused {fused_mode}", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(cfg, layers)
    line = {
        "metric": "decode-attn us/layer-step (append + split-K attention) + achieved HBM GB/s",
        "value": round(us_layer, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (int4/int8 codes)",
        "data": "synthetic (seeded; distinct cache per layer)",
        "config": {
            "workload": cfg.name,
            "config_index": cfg.index,
            "batch": cfg.batch,
            "q_heads": cfg.q_heads,
            "kv_heads": cfg.kv_heads,
            "layers": nl,
            "model_layers": cfg.layers,
            "context": ctx,
            "kv_format": f"K {cfg.k_format} / V {cfg.v_format} g32"
                         + (" + 4 fp16 K channels" if cfg.outlier_channels else ""),
            "chunk_tokens": layers[0].plan.chunk_tokens,
            "hip_graph": use_graph,
            "launch": used,
            "us_per_layer_step_by_launch": {k: round(v * 1000.0 / nl, 3) for k, v in ms_by.items()},
            "fused_step": fused,
        },
        "attention_us_per_layer_step": None if us_attn is None else round(us_attn, 3),
        "append_us_per_layer_step": None if us_app is None else round(us_app, 3),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "frac_of_stream_read": (None if ceiling is None
                                    else round(achieved / ceiling["read_GBps_same_bytes"], 4)),
            "traffic": measured_traffic(cfg.index),
            "bytes_per_launch": roof_bytes,
            "kernel": (attention_kernels(cfg, layers[0]) +
                       (" with the append fused (one kvq_append_decode_attn call per layer)"
                        if fused else " (one kvq_decode_attn call per layer)")),
        },
        "stream_ceiling": ceiling,
        "engine_api": eng,
        "int4_fused": fused_mode,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
