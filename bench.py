"""Benchmark: the 311M-parameter GPT training step (config 3) on one MI355X.

Workload (the configuration the metric is quoted on):
24 layers, hidden 1024, 16 heads (MHA, head_dim 64), SwiGLU ffn 2736, vocab 8192
tied, bf16 parameters and activations with fp32 master weights and AdamW
(lr 3e-4, betas (0.9, 0.95), eps 1e-8, weight decay 0.1, grad-norm clip 1.0),
micro-batch 16 x seq 512 of uniform random tokens resident in HBM, full
per-layer activation recompute.  One step = forward + backward + clip +
optimizer update.  The same step without checkpointing gives the recompute
overhead.

Prints ONE JSON line.  ``value`` = tokens/s of the full-recompute step.
``roofline`` is measured live with HIP events on the launch stream for each
hand-written kernel at the config-3 shapes (``kernels``); the dominant one
(largest time per training step) is ``roofline``.  ``cpu_baseline`` times the
CPU oracle (the repo's PyTorch-CPU restatement) on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "train tokens/s + peak act GB/layer, 311M seq512 recompute, 1 MI355X; HBM/MFMA %"

C3 = dict(layers=24, hidden_size=1024, ffn_hidden_size=2736, heads=16, seq_length=512,
          vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
BATCH, SEQ = 16, 512
# GQA variant and one ring rank's attention share
C4 = dict(layers=16, hidden_size=2048, ffn_hidden_size=5632, heads=32, kv_heads=8, seq_length=2048,
          vocab_size=8192, norm_epsilon=1e-5, rope_theta=1e4)
C4_BATCH, C4_SEQ = 4, 2048


def parse() -> argparse.Namespace:
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-kernels", action="store_true", help="skip the per-kernel roofline timing")
    p.add_argument("--no-eager", action="store_true", help="skip the no-checkpoint comparison run")
    p.add_argument("--no-legs", action="store_true",
                   help="skip the config-4, config-5, PyTorch and vendor-GEMM legs of the default line")
    p.add_argument("--no-torch", action="store_true",
                   help="skip the plain PyTorch-ROCm implementation of the same step (context)")
    p.add_argument("--host-launch", action="store_true",
                   help="time the steps with every kernel launched from the host (no HIP graph)")
    p.add_argument("--only-kernels", action="store_true", help="time the kernels only (for profiling)")
    p.add_argument("--kernel", default=None, help="with --only-kernels: time just this kernel")
    p.add_argument("--config", default="c3", choices=("c3", "c4", "c5"),
                   help="c3: the metric's 311M step (default); c4: the GQA step; c5: one ring rank's attention")
    p.add_argument("--metrics-jsonl", default=None,
                   help="append the timed interval as one train record of the reference's metric history")
    return p.parse_args()


def run_steps(mode: str, steps: int, warmup: int, device, metrics_jsonl: str | None = None,
              model_cfg: dict = C3, batch: int = BATCH, seq: int = SEQ, graph: bool = True) -> dict:
    """Eager steps, then (``graph``) the same step captured as a HIP graph and
    replayed (``CapturedTrainStep``): both timed, the graph's time reported."""
    import torch

    import nano_megatron_amd as nm

    torch.manual_seed(1234)
    cfg = nm.GPTConfig(**model_cfg)
    model = nm.GPTModel(cfg, activation_checkpoint_config=nm.ActivationCheckpointConfig(mode=mode))
    model = model.to(device=device, dtype=torch.bfloat16).train()
    from nano_megatron_amd.optim import MasterAdamW

    opt = MasterAdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                      clip_grad_norm=1.0)
    g = torch.Generator(device=device).manual_seed(1234)
    ids = torch.randint(0, cfg.vocab_size, (batch, seq + 1), device=device, generator=g)
    x, y = ids[:, :seq].contiguous(), ids[:, 1:].contiguous()

    def step():
        opt.zero_grad()
        loss = model(x, labels=y).loss
        loss.backward()
        opt.step()
        return loss.detach()  # no reference to the step's autograd graph outlives it

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # Activation memory (training/trainer.py:583-585, 752-776 definitions): with
    # the gradients of the previous step kept allocated (zeroed in place), the
    # peak during forward+backward minus what was resident at its start, and the
    # memory the forward leaves saved for the backward.
    for p in opt.params:
        p.grad = torch.zeros_like(p)
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    start_alloc = torch.cuda.memory_allocated()
    out = model(x, labels=y)
    torch.cuda.synchronize()
    saved_after_fwd = torch.cuda.memory_allocated() - start_alloc
    out.loss.backward()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - start_alloc
    del out
    opt.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    elapsed = eager_elapsed = time.perf_counter() - t0
    launch = "eager"
    if graph:
        from nano_megatron_amd.graph import CapturedTrainStep

        cap = CapturedTrainStep(model, opt, x, y)
        for _ in range(2):
            cap.step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = cap.step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        launch = "hip_graph"
    if metrics_jsonl:
        from nano_megatron_amd import metrics as M

        m = M.train_metrics(loss=float(loss.item()), learning_rate=3e-4, samples=batch * steps,
                            tokens=batch * seq * steps, seconds=elapsed,
                            grad_norm=float(opt.last_grad_norm), device=device)
        with open(metrics_jsonl, "a") as f:
            f.write(M.history_line(sequence=0, step=warmup + 1 + steps, prefix="train", metrics=m,
                                   consumed_samples=batch * (warmup + 1 + steps),
                                   consumed_tokens=batch * seq * (warmup + 1 + steps)) + "\n")
    result = dict(
        ms_per_step=1e3 * elapsed / steps,
        tokens_per_s=batch * seq * steps / elapsed,
        launch=launch,
        eager_ms_per_step=1e3 * eager_elapsed / steps,
        eager_tokens_per_s=batch * seq * steps / eager_elapsed,
        loss=float(loss.item()),
        peak_act_gib_per_layer=peak / cfg.layers / 2**30,
        saved_act_mib_per_layer=saved_after_fwd / cfg.layers / 2**20,
    )
    del model, opt, x, y, ids
    torch.cuda.empty_cache()
    return result


def block_saved_mib(mode: str, device, model_cfg: dict = C3, batch: int = BATCH, seq: int = SEQ) -> float:
    """Activation memory one block leaves saved for the backward: what a forward
    of a 2-layer model keeps allocated minus what a 1-layer model keeps, at the
    configuration's width and batch (the embedding, final norm and LM head keep
    the same in both, so the difference is one block's share)."""
    import torch

    import nano_megatron_amd as nm

    saved = []
    for layers in (1, 2):
        torch.manual_seed(1234)
        cfg = nm.GPTConfig(**{**model_cfg, "layers": layers})
        model = nm.GPTModel(cfg, activation_checkpoint_config=nm.ActivationCheckpointConfig(mode=mode))
        model = model.to(device=device, dtype=torch.bfloat16).train()
        g = torch.Generator(device=device).manual_seed(1234)
        ids = torch.randint(0, cfg.vocab_size, (batch, seq + 1), device=device, generator=g)
        x, y = ids[:, :seq].contiguous(), ids[:, 1:].contiguous()
        # a first forward packs the block weights into the fused path's layout
        # (new storage, old freed), which must not count as saved activation
        model(x, labels=y)
        torch.cuda.synchronize()
        start = torch.cuda.memory_allocated()
        out = model(x, labels=y)
        torch.cuda.synchronize()
        saved.append(torch.cuda.memory_allocated() - start)
        del out, model, x, y, ids
        torch.cuda.empty_cache()
    return (saved[1] - saved[0]) / 2**20


INFINITY_CACHE_BYTES = 256 << 20  # MI355X last-level (MALL) cache


def _input_sets(nbytes: int) -> int:
    """How many input sets an HBM-bound kernel's timing rotates through: enough
    that between two launches on one set the others touch more than twice the
    256 MB Infinity Cache, so each launch reads its inputs from HBM."""
    return max(2, min(24, math.ceil(2 * INFINITY_CACHE_BYTES / max(nbytes, 1)) + 1))


def kernel_rooflines(device, only: str | None = None) -> list[dict]:
    """Average launch time (HIP events on the launch stream) of each hand-written
    kernel at the config-3 shapes, with algorithmic bytes / FLOPs per launch
    (``only``: just the named one).  HBM-bound kernels rotate through input
    sets larger than the Infinity Cache (``_input_sets``); MFMA-bound ones run
    on one set, as in the step, where their operands were just written."""
    import torch

    import nano_megatron_amd as nm
    from nano_megatron_amd import functional as Fn
    from nano_megatron_amd.optim import MasterAdamW

    T, H, F, V = BATCH * SEQ, C3["hidden_size"], C3["ffn_hidden_size"], C3["vocab_size"]
    nh, d = C3["heads"], C3["hidden_size"] // C3["heads"]
    L = C3["layers"]
    g = torch.Generator(device=device).manual_seed(1)
    bf = torch.bfloat16

    def randn(*shape, scale=1.0):
        return (scale * torch.randn(*shape, device=device, generator=g)).to(bf)

    tab = nm.RotaryEmbedding(d).tables(device, SEQ)
    causal_flops = 2 * 2 * BATCH * nh * SEQ * SEQ * d / 2
    E = 2  # bytes per bf16 element
    chunk = 2048

    # --- HBM-bound kernels: make() allocates one input set and returns its launch
    def mk_rms_fwd():
        x, w = randn(T, H), (1 + randn(H, scale=0.02).float()).to(bf)
        y = torch.empty_like(x)
        return lambda: Fn._lib.call("nmb_rmsnorm_fwd", x.data_ptr(), w.data_ptr(), y.data_ptr(), None, T, H,
                                    1e-5, Fn._lib.NMB_BF16, Fn._lib.stream_of(x))

    def mk_rms_bwd():
        x, w, dy, dres = randn(T, H), (1 + randn(H, scale=0.02).float()).to(bf), randn(T, H), randn(T, H)
        dx, dw = torch.empty_like(x), torch.empty_like(w)
        nb = Fn._lib.ctypes.c_size_t(0)
        Fn._lib.call("nmb_rmsnorm_bwd_workspace_bytes", T, H, Fn._lib.ctypes.byref(nb))
        ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=device)
        return lambda: Fn._lib.call("nmb_rmsnorm_bwd", x.data_ptr(), w.data_ptr(), dy.data_ptr(), dres.data_ptr(),
                                    dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws.numel(), T, H, 1e-5,
                                    Fn._lib.NMB_BF16, Fn._lib.stream_of(x))

    def mk_rope():
        q = randn(BATCH, SEQ, nh, d)
        out = torch.empty_like(q)
        return lambda: Fn.rope_apply(q, out, tab.cos, tab.sin)

    def mk_dropout_add():
        x, r = randn(T, H), randn(T, H)
        out = torch.empty_like(x)
        return lambda: Fn._lib.call("nmb_dropout_add", x.data_ptr(), r.data_ptr(), out.data_ptr(), T * H, 0.1,
                                    1234, Fn._lib.NMB_BF16, Fn._lib.stream_of(x))

    def mk_swiglu_fwd():
        gu, act = randn(T, 2 * F), torch.empty(T, F, dtype=bf, device=device)
        return lambda: Fn.swiglu_fwd(gu[:, :F], gu[:, F:], act)

    def mk_swiglu_bwd():
        gu, dh = randn(T, 2 * F), randn(T, F)
        dgu, act = torch.empty_like(gu), torch.empty(T, F, dtype=bf, device=device)
        return lambda: Fn.swiglu_bwd(gu[:, :F], gu[:, F:], dh, dgu[:, :F], dgu[:, F:], act)

    def mk_ce_fwd():
        logits = randn(chunk, V)
        targets = torch.randint(0, V, (chunk,), device=device, generator=g)
        loss = torch.empty(chunk, dtype=torch.float32, device=device)
        lse_c = torch.empty_like(loss)
        return lambda: Fn.ce_fwd(logits, targets, -100, loss, lse_c)

    def mk_ce_bwd():
        logits = randn(chunk, V)
        targets = torch.randint(0, V, (chunk,), device=device, generator=g)
        loss = torch.empty(chunk, dtype=torch.float32, device=device)
        lse_c = torch.empty_like(loss)
        Fn.ce_fwd(logits, targets, -100, loss, lse_c)
        grad_c = torch.full((chunk,), 1.0 / T, device=device)
        # in place: the values drift over launches, the work per launch does not
        return lambda: Fn.ce_bwd_(logits, targets, -100, lse_c, grad_c)

    def mk_emb_fwd():
        table = randn(V, H, scale=0.02)
        ids = torch.randint(0, V, (T,), device=device, generator=g)
        out = torch.empty(T, H, dtype=bf, device=device)
        return lambda: Fn._lib.call("nmb_embedding_fwd", table.data_ptr(), ids.data_ptr(), out.data_ptr(), T, V,
                                    H, Fn._lib.NMB_BF16, Fn._lib.stream_of(table))

    def mk_emb_bwd():
        dout = randn(T, H)
        ids = torch.randint(0, V, (T,), device=device, generator=g)
        lm_grad, grad = randn(V, H), torch.empty(V, H, dtype=bf, device=device)
        return lambda: Fn._lib.call("nmb_embedding_bwd", dout.data_ptr(), ids.data_ptr(), lm_grad.data_ptr(),
                                    grad.data_ptr(), T, V, H, Fn._lib.NMB_BF16, Fn._lib.stream_of(dout))

    # --- MFMA-bound kernels: one input set
    qkv = randn(T, 3 * H)
    q = qkv[:, :H].view(BATCH, SEQ, nh, d)
    k = qkv[:, H:2 * H].view(BATCH, SEQ, nh, d)
    v = qkv[:, 2 * H:].view(BATCH, SEQ, nh, d)
    o, lse = Fn.attn_fwd_bshd(q, [k], [v], (0,), causal=True, q_offset=0, scale=None)
    do = randn(BATCH, SEQ, nh, d)
    dqkv = torch.empty_like(qkv)
    dq = dqkv[:, :H].view(BATCH, SEQ, nh, d)
    dk = dqkv[:, H:2 * H].view(BATCH, SEQ, nh, d)
    dv = dqkv[:, 2 * H:].view(BATCH, SEQ, nh, d)
    x = randn(T, H)
    act = torch.empty(T, F, dtype=bf, device=device)

    def gemm_case(name, m, n, k_, a_t, b_t, per_step, residual=False):
        a = randn(k_, m).t() if a_t else randn(m, k_)
        b = randn(k_, n) if b_t else randn(n, k_).t()
        c = randn(m, n) if residual else None
        out = torch.empty(m, n, dtype=bf, device=device)
        fn = (lambda: Fn.mm(a, b, out=out, c=c, beta=1.0)) if residual else (lambda: Fn.mm(a, b, out=out))
        nbytes = (m * k_ + k_ * n + m * n * (2 if residual else 1)) * E
        return (name, fn, nbytes, 2.0 * m * n * k_, "mfma", per_step)

    w_qkv = randn(3 * H, H)
    qkv_out = torch.empty(T, 3 * H, dtype=bf, device=device)
    w_gu = randn(2 * F, H)
    dy_swb, wd_swb, gu_swb = randn(T, H), randn(H, F), randn(T, 2 * F)
    g_de, x_de = randn(chunk, V), randn(chunk, H)
    de32 = torch.zeros(V, H, dtype=torch.float32, device=device)
    gu_buf = torch.empty(T, 2 * F, dtype=bf, device=device)
    gemms = [
        # the Q/K/V projection with RoPE of q and k in its epilogue, as the block runs it
        ("gemm_qkv_rope",
         lambda: Fn.mm_rope(x, w_qkv.t(), seq=SEQ, head_dim=d, rope_cols=2 * H, cos=tab.cos, sin=tab.sin,
                            out=qkv_out),
         (T * H + 3 * H * H + 3 * T * H) * E, 2.0 * T * 3 * H * H, "mfma", 2 * L),
        gemm_case("gemm_o_residual", T, H, H, False, False, 2 * L, residual=True),
        # the gate/up projection: the forward's applies SwiGLU in its epilogue; the
        # product [g|u] alone (same kernel and plan) is what a block without
        # checkpointing keeps (not in the full-recompute step)
        ("gemm_gate_up", lambda: Fn.mm_gate_up(x, w_gu, act=False, gu=True, gu_out=gu_buf),
         (T * H + 2 * F * H + 2 * T * F) * E, 2.0 * T * 2 * F * H, "mfma", 0),
        ("gemm_gate_up_swiglu", lambda: Fn.mm_gate_up(x, w_gu, act=True, act_out=act),
         (T * H + 2 * F * H + T * F) * E, 2.0 * T * 2 * F * H, "mfma", L),
        gemm_case("gemm_down_residual", T, H, F, False, False, L, residual=True),
        # the recomputed block's MLP backward in one kernel: [g|u] = n2 [Wg;Wu]^T
        # and ds = dY Wd per tile, the SwiGLU backward on both, [dg|du] and the
        # re-emitted activation written; neither [g|u] nor ds reaches memory
        ("gemm_gate_up_swiglu_bwd", lambda: Fn.mm_gate_up_swiglu_bwd(x, w_gu, dy_swb, wd_swb),
         (2 * T * H + 2 * F * H + H * F + 3 * T * F) * E, 2.0 * T * 2 * F * H + 2.0 * T * F * H, "mfma", L),
        # ds = dY Wd with the SwiGLU backward as its epilogue, reading a kept [g|u]
        # (a block without checkpointing; not in the full-recompute step)
        ("gemm_d_swiglu_bwd", lambda: Fn.mm_swiglu_bwd(dy_swb, wd_swb, gu_swb),
         (T * H + H * F + 5 * T * F) * E, 2.0 * T * F * H, "mfma", 0),
        gemm_case("gemm_dw_down", H, F, T, True, True, L),
        gemm_case("gemm_d_norm2", T, H, 2 * F, False, True, L),
        gemm_case("gemm_dw_gate_up", 2 * F, H, T, True, True, L),
        gemm_case("gemm_d_attn_out", T, H, H, False, True, L),
        gemm_case("gemm_dw_o", H, H, T, True, True, L),
        gemm_case("gemm_d_norm1", T, H, 3 * H, False, True, L),
        gemm_case("gemm_dw_qkv", 3 * H, H, T, True, True, L),
        gemm_case("gemm_lm_logits", chunk, V, H, False, False, 2 * T // chunk),
        gemm_case("gemm_lm_dx", chunk, H, V, False, True, T // chunk),
        # the tied table gradient: dE += G^T x over the token chunks, summed in fp32
        ("gemm_lm_dE", lambda: Fn.mm_f32out(g_de.t(), x_de, de32, beta=1.0),
         (chunk * V + chunk * H) * E + 2 * V * H * 4, 2.0 * V * H * chunk, "mfma", T // chunk),
    ]
    hbm = [
        # name, make, algorithmic bytes, launches per training step (full recompute)
        ("rmsnorm_fwd", mk_rms_fwd, 2 * T * H * E + H * E, 4 * L + 1),
        # in the block the norm backward also adds the residual branch's gradient;
        # the launch includes the dw column sum
        ("rmsnorm_bwd", mk_rms_bwd, 4 * T * H * E + 2 * H * E, 2 * L + 1),
        # the standalone rotary kernel; the step fuses RoPE into the QKV GEMM and the attention backward
        ("rope_apply", mk_rope, 2 * T * H * E, 0),
        # residual + dropout (p 0.1) on [T, H]; the configurations train at dropout 0
        ("dropout_add", mk_dropout_add, 3 * T * H * E, 0),
        # the standalone activation; the checkpointed step fuses it into the gate/up GEMM
        ("swiglu_fwd", mk_swiglu_fwd, 3 * T * F * E, 0),
        # the standalone backward; the step runs it as the down projection's dX GEMM epilogue
        ("swiglu_bwd", mk_swiglu_bwd, 6 * T * F * E, 0),
        ("ce_fwd", mk_ce_fwd, chunk * V * E + chunk * 16, T // chunk),
        ("ce_bwd", mk_ce_bwd, 2 * chunk * V * E + chunk * 16, T // chunk),
        # token rows gathered and written; the backward reads the output gradient and the
        # tied LM head's table gradient once and writes the table gradient once
        ("embedding_fwd", mk_emb_fwd, 2 * T * H * E + T * 8, 1),
        ("embedding_bwd", mk_emb_bwd, T * H * E + 2 * V * H * E + T * 8, 1),
    ]
    cases = [(name, make, nbytes, 0, "hbm", per) for name, make, nbytes, per in hbm]
    # attention at S 512 / D 64 sits below the ridge (127 FLOP/B forward, 159
    # backward, against ~312 for 2.5 PFLOP/s over 8 TB/s), so its roofline is
    # HBM: compulsory bytes over time; the FLOP rate is reported beside it
    cases += [
        ("attn_fwd", lambda: Fn.attn_fwd_bshd(q, [k], [v], (0,), causal=True, q_offset=0, scale=None, out=o,
                                              lse=lse),
         4 * T * H * E + BATCH * nh * SEQ * 4, causal_flops, "hbm", 2 * L),
        ("attn_fwd_from_lse", lambda: Fn.attn_fwd_from_lse_bshd(q, [k], [v], (0,), lse, causal=True, q_offset=0,
                                                                scale=None, out=o),
         4 * T * H * E + BATCH * nh * SEQ * 4, causal_flops, "hbm", 0),
        # the backward with the inverse RoPE of dq and dk in its stores, as the block runs it
        ("attn_bwd_rope", lambda: Fn.attn_bwd_rope_bshd(q, k, v, o, do, lse, dq, dk, dv, causal=True, q_offset=0,
                                                        scale=None, cos=tab.cos, sin=tab.sin),
         8 * T * H * E + BATCH * nh * SEQ * 4, 2.5 * causal_flops, "hbm", L),
    ] + gemms
    names = [c_[0] for c_ in cases] + ["adamw_step"]
    if only is not None and only not in names:
        raise SystemExit(f"bench.py: no kernel named {only!r}")
    out = []
    side = torch.cuda.Stream(device)
    stream = torch.cuda.current_stream(device)

    def record(name, us, nbytes, flops, bound, per_step, sets):
        gbs = nbytes / us / 1e3
        entry = dict(kernel=name, us=round(us, 2), bytes=int(nbytes), gbs=round(gbs, 1),
                     hbm_frac=round(gbs / HBM_PEAK_GBS, 3), bound=bound,
                     us_per_step=round(us * per_step, 1), launches_per_step=per_step, input_sets=sets)
        if flops:
            tf = flops / us / 1e6
            entry.update(flops=int(flops), tflops=round(tf, 1), mfma_frac=round(tf / BF16_PEAK_TFLOPS, 4))
        out.append(entry)

    def time_launches(fns, sets):
        # launches captured in a HIP graph and replayed: the events then time GPU
        # work only, not the host cost of issuing each launch
        n = sets * max(1, math.ceil(20 / sets))
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            for f in fns:
                f()
        stream.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(n):
                fns[i % sets]()
        graph.replay()
        torch.cuda.synchronize()
        # three rounds of five replays; the best round's average per launch
        # (the clocks of a box vary between rounds by up to ~15%)
        reps, rounds = 5, 3
        us = float("inf")
        for _ in range(rounds):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(reps):
                graph.replay()
            end.record(stream)
            end.synchronize()
            us = min(us, start.elapsed_time(end) * 1e3 / (n * reps))
        del graph
        return us

    def mk_copy(nbytes):
        # a plain device copy moving the same bytes (half read, half written)
        def make():
            src = torch.empty(max(nbytes // 2, 1), dtype=torch.uint8, device=device).fill_(1)
            dst = torch.empty_like(src)
            return lambda: dst.copy_(src)
        return make

    for name, fn, nbytes, flops, bound, per_step in cases:
        if only is not None and name != only:
            continue
        sets = 1
        fns = [fn]
        if bound == "hbm" and not flops:
            sets = _input_sets(nbytes)
            fns = [fn() for _ in range(sets)]
        us = time_launches(fns, sets)
        del fns
        record(name, us, nbytes, flops, bound, per_step, sets)
        if bound == "hbm":
            # the same bytes moved by a plain copy, timed the same way: the
            # ceiling at this transfer size (launch ramp and tail included)
            cfns = [mk_copy(nbytes)() for _ in range(_input_sets(nbytes))]
            cus = time_launches(cfns, len(cfns))
            del cfns
            out[-1].update(same_size_copy_us=round(cus, 2), same_size_copy_frac=round(cus / us, 3))

    if only is None or only == "adamw_step":
        # the optimizer of the step: global grad-norm clip + fp32-master AdamW over the
        # 310.8M parameters of config 3 in the model's tensor shapes (8.7 GB per launch,
        # far beyond the cache); timed eagerly (each launch is ~1.7 ms)
        shapes = [(V, H)] + [(H,), (3 * H, H), (H, H), (H,), (2 * F, H), (H, F)] * L + [(H,)]
        params = [torch.nn.Parameter(randn(*sh, scale=0.02)) for sh in shapes]
        for p_ in params:
            p_.grad = randn(*p_.shape, scale=1e-3)
        opt = MasterAdamW(params, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, clip_grad_norm=1.0)
        n_el = sum(p_.numel() for p_ in params)
        for _ in range(3):
            opt.step()
        torch.cuda.synchronize()
        us = float("inf")
        for _ in range(3):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(5):
                opt.step()
            end.record(stream)
            end.synchronize()
            us = min(us, start.elapsed_time(end) * 1e3 / 5)
        # 28 B per parameter: bf16 grad read, bf16 param written, fp32 master and two
        # moments read and written (the norm pass's second read of the grads not counted)
        record("adamw_step", us, 28 * n_el, 0, "hbm", 1, 1)
        del opt, params
        torch.cuda.empty_cache()
    return out


def measured_traffic(kernel: str) -> int | None:
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter
    summary ``profiles/<kernel>_c3_traffic.md`` (FETCH_SIZE + WRITE_SIZE, each
    scaled by the same counter's reading for a copy of known size), if any."""
    path = os.path.join(ROOT, "profiles", f"{kernel}_c3_traffic.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    return None


def measured_ceilings(device) -> dict:
    """Achievable ceilings on this box, beside the datasheet peaks: a plain
    256 MiB device copy (256 MiB read + 256 MiB written) and an 8192^3 bf16
    product (A row-major, B = W^T of a row-major W) by this library's GEMM and
    by torch (hipBLASLt).  Best of three rounds of ten launches each."""
    import torch

    from nano_megatron_amd import functional as Fn

    def best_ms(fn, reps=10, rounds=3):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(rounds):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(reps):
                fn()
            end.record()
            end.synchronize()
            best = min(best, start.elapsed_time(end) / reps)
        return best

    bf = torch.bfloat16
    n = 128 << 20  # bf16 elements: 256 MiB
    src = torch.ones(n, dtype=bf, device=device)
    dst = torch.empty_like(src)
    copy_ms = best_ms(lambda: dst.copy_(src))
    copy_gbs = 2 * n * 2 / (copy_ms * 1e-3) / 1e9
    del src, dst
    g = torch.Generator(device=device).manual_seed(7)
    m = 8192
    a = torch.randn(m, m, device=device, dtype=bf, generator=g)
    w = torch.randn(m, m, device=device, dtype=bf, generator=g)
    out = torch.empty(m, m, device=device, dtype=bf)
    flops = 2.0 * m * m * m
    ours = flops / (best_ms(lambda: Fn.mm(a, w.t(), out=out)) * 1e-3) / 1e12
    lt = flops / (best_ms(lambda: torch.mm(a, w.t(), out=out)) * 1e-3) / 1e12
    return dict(copy_256mib_gbs=round(copy_gbs, 1), copy_hbm_frac=round(copy_gbs / HBM_PEAK_GBS, 3),
                gemm_8192_tflops=round(ours, 1), gemm_8192_mfma_frac=round(ours / BF16_PEAK_TFLOPS, 3),
                hipblaslt_gemm_8192_tflops=round(lt, 1))


def copy_calibration(device) -> None:
    """A plain device copy of 256 MiB (read 256 MiB, write 256 MiB), run once so
    that a counter pass sees the HBM bytes one such copy reports."""
    import torch

    src = torch.empty(128 << 20, dtype=torch.bfloat16, device=device).fill_(1.0)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def _host_cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float = 25.0) -> dict:
    """The repo's own CPU path (the oracle's PyTorch-CPU restatement of the
    reference modules, fp32) running the full 24-layer config-3 training step
    on one 512-token sequence: forward with per-layer recompute, backward,
    global-norm clip and AdamW (torch.optim.AdamW, the reference's fp32 mode,
    data_parallel/_common.py:242-252), timed with perf_counter after one
    warm-up step; the median of at least three steps, or as many as fit in
    ``seconds``.  Runs on every core the host reports
    (``torch.set_num_threads(os.cpu_count())``); reports the core count, the
    threads used, the cores this process may run on (affinity) and the
    implied FLOP rate, and the batch in its own fields."""
    import torch

    from oracle import reference as R

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    threads = torch.get_num_threads()
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else cores

    class Ck:
        mode = "full"
        block_interval = 1

    class Cfg:
        pass

    for k_, v_ in C3.items():
        setattr(Cfg, k_, v_)
    torch.manual_seed(0)
    model = R.OracleGPTModel(Cfg(), activation_checkpoint_config=Ck()).train()
    opt = torch.optim.AdamW(model.parameters(), lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    g = torch.Generator().manual_seed(1234)
    ids = torch.randint(0, C3["vocab_size"], (1, SEQ + 1), generator=g)
    x, y = ids[:, :SEQ], ids[:, 1:]

    def step() -> float:
        t0 = time.perf_counter()
        opt.zero_grad(set_to_none=True)
        model(x, labels=y).loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        return time.perf_counter() - t0

    warm = step()
    times = []
    while len(times) < 3 or (sum(times) + warm < seconds and len(times) < 9):
        times.append(step())
    times.sort()
    t_step = times[len(times) // 2]
    flops = model_step_flops(C3, 1, SEQ, recompute=True)
    del model, opt
    return dict(
        value=round(SEQ / t_step, 1),
        unit="tokens/s",
        cores=cores,
        threads=threads,
        cores_usable=usable,
        kind="port",
        dtype="f32",
        batch=1,
        seq_len=SEQ,
        tokens_per_step=SEQ,
        gpu_batch=BATCH,
        sample=(f"CPU oracle (PyTorch fp32, {threads} threads on {cores} cores of {_host_cpu_model()}): the full 24-layer "
                f"config-3 step (forward with per-layer recompute, backward, clip, AdamW) on one "
                f"512-token sequence, median of {len(times)} steps after one warm-up: "
                f"{t_step:.2f} s per step ({min(times):.2f}-{max(times):.2f} s), "
                f"{flops / t_step / 1e9:.0f} GFLOP/s implied"),
        step_s=round(t_step, 3),
        steps_timed=len(times),
        implied_gflops=round(flops / t_step / 1e9, 1),
    )


def model_step_flops(cfg: dict, batch: int, seq: int, recompute: bool) -> float:
    """FLOPs of one training step (GEMMs, causal attention, LM head): per layer
    3x the forward GEMMs (forward, dX, dW) and 3.5x the causal attention forward
    (forward 1x, backward 2.5x), plus 3x the LM head; recompute adds one forward
    without the down projection."""
    t, h, f, v = batch * seq, cfg["hidden_size"], cfg["ffn_hidden_size"], cfg["vocab_size"]
    hq = cfg["heads"]
    hkv = cfg.get("kv_heads") or hq
    d = h // hq
    gemm = 2 * t * (h * hq * d + 2 * h * hkv * d + hq * d * h + 3 * h * f)
    attn = 2 * batch * hq * seq * seq * d  # causal forward (half of the 4 b h s^2 d)
    total = cfg["layers"] * (3 * gemm + 3.5 * attn) + 3 * 2 * t * h * v
    if recompute:
        total += cfg["layers"] * (gemm - 2 * t * h * f + attn)
    return total


def c4_leg(args, device, eager: bool = True) -> dict:
    """Config 4: the GQA step, full recompute and none."""
    full = run_steps("full", args.steps, args.warmup, device, None, C4, C4_BATCH, C4_SEQ,
                     graph=not args.host_launch)
    print("c4 full: " + json.dumps(full), file=sys.stderr, flush=True)
    fl = model_step_flops(C4, C4_BATCH, C4_SEQ, recompute=True)
    tf = fl / (full["ms_per_step"] * 1e-3) / 1e12
    leg = dict(
        workload="C4: GQA GPT (16L, H2048, 32 query / 8 KV heads D64, ffn 5632, vocab 8192 tied) training "
                 "step, B4 x S2048, full per-layer recompute, bf16 + fp32-master AdamW",
        tokens_per_s=round(full["tokens_per_s"], 1), ms_per_step=round(full["ms_per_step"], 3),
        launch=full["launch"], host_launched_tokens_per_s=round(full["eager_tokens_per_s"], 1),
        model_tflops=round(tf, 1), mfma_frac=round(tf / BF16_PEAK_TFLOPS, 4),
        peak_act_gib_per_layer=round(full["peak_act_gib_per_layer"], 4),
        # one block's saved activation (2-layer minus 1-layer model); the
        # whole-model figure spreads the head's saved state over the layers
        saved_act_mib_per_layer=round(block_saved_mib("full", device, C4, C4_BATCH, C4_SEQ), 2),
        act_floor_mib_per_layer=32.0,
        saved_act_mib_whole_model_per_layer=round(full["saved_act_mib_per_layer"], 2),
        loss=round(full["loss"], 4),
    )
    if eager:
        none = run_steps("none", args.steps, args.warmup, device, None, C4, C4_BATCH, C4_SEQ,
                         graph=not args.host_launch)
        print("c4 none: " + json.dumps(none), file=sys.stderr, flush=True)
        leg["no_checkpoint_tokens_per_s"] = round(none["tokens_per_s"], 1)
        leg["recompute_overhead"] = round(full["ms_per_step"] / none["ms_per_step"] - 1.0, 4)
    return leg


def vendor_gemm_leg(device, calls: int = 20, rounds: int = 3) -> dict:
    """This library's bf16 GEMM against ``torch.mm`` (the vendor BLAS that torch
    picks on ROCm) on the twelve plain product shapes of the config-3 step
    (forward, dX and weight-gradient products; the epilogue variants run as
    plain products here so that both sides do the same work), same operand
    views, best of ``rounds`` rounds of ``calls`` calls each, HIP events on the
    current stream."""
    import torch

    from nano_megatron_amd import functional as Fn

    bf = torch.bfloat16
    gen = torch.Generator(device=device).manual_seed(0)
    T, H, F = BATCH * SEQ, C3["hidden_size"], C3["ffn_hidden_size"]

    def randn(*shape):
        return (0.05 * torch.randn(*shape, device=device, generator=gen)).to(bf)

    # (name, M, N, K, A stored transposed, B stored [K, N])
    cases = [("qkv", T, 3 * H, H, False, False), ("o", T, H, H, False, False),
             ("gate_up", T, 2 * F, H, False, False), ("down", T, H, F, False, False),
             ("d_swiglu", T, F, H, False, True), ("d_norm2", T, H, 2 * F, False, True),
             ("d_attn_out", T, H, H, False, True), ("d_norm1", T, H, 3 * H, False, True),
             ("dw_gate_up", 2 * F, H, T, True, True), ("dw_down", H, F, T, True, True),
             ("dw_o", H, H, T, True, True), ("dw_qkv", 3 * H, H, T, True, True)]

    def best_us(fn):
        best = None
        for _ in range(rounds):
            for _ in range(3):
                fn()
            torch.cuda.synchronize(device)
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(calls):
                fn()
            e.record()
            torch.cuda.synchronize(device)
            t = s.elapsed_time(e) / calls * 1e3
            best = t if best is None else min(best, t)
        return best

    shapes, ours_sum, torch_sum = [], 0.0, 0.0
    for name, m, n, k, a_t, b_t in cases:
        a = randn(k, m).t() if a_t else randn(m, k)
        b = randn(k, n) if b_t else randn(n, k).t()
        out, ref = torch.empty(m, n, dtype=bf, device=device), torch.empty(m, n, dtype=bf, device=device)
        ours = best_us(lambda: Fn.mm(a, b, out=out))
        theirs = best_us(lambda: torch.mm(a, b, out=ref))
        ours_sum, torch_sum = ours_sum + ours, torch_sum + theirs
        shapes.append(dict(name=name, m=m, n=n, k=k, ours_us=round(ours, 2), torch_us=round(theirs, 2),
                           max_abs_diff=float((out.float() - ref.float()).abs().max())))
        del a, b, out, ref
    return dict(workload="the config-3 step's plain GEMM shapes, this library against torch.mm",
                ours_us_sum=round(ours_sum, 1), torch_us_sum=round(torch_sum, 1),
                ratio=round(ours_sum / torch_sum, 3), shapes=shapes)


def torch_eager_leg(device, steps: int = 10, warmup: int = 3) -> dict:
    """The config-3 step written in plain PyTorch on the same GPU, for context:
    the reference's modules as torch operations (F.rms_norm, RoPE by tensor
    ops, SDPA causal attention, nn.Linear on hipBLASLt, SwiGLU, the full-logit
    cross-entropy, torch's non-reentrant checkpoint per layer), bf16 parameters
    with an fp32 master copy stepped by torch's fused AdamW after a global
    clip (the ZeRO path's arithmetic at one rank), launched from the host.
    Same shapes, same work per step; random weights of the same sizes."""
    import torch
    import torch.nn.functional as F
    from torch import nn
    from torch.utils.checkpoint import checkpoint

    L, H, nh, ff, V = C3["layers"], C3["hidden_size"], C3["heads"], C3["ffn_hidden_size"], C3["vocab_size"]
    B, S, d = BATCH, SEQ, C3["hidden_size"] // C3["heads"]

    class Layer(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.n1, self.n2 = nn.Parameter(torch.ones(H)), nn.Parameter(torch.ones(H))
            self.q, self.k, self.v, self.o = (nn.Linear(H, H, bias=False) for _ in range(4))
            self.g, self.u = nn.Linear(H, ff, bias=False), nn.Linear(H, ff, bias=False)
            self.d = nn.Linear(ff, H, bias=False)

        def forward(self, x, cos, sin):
            def rope(t):
                a, b = t.chunk(2, -1)
                return t * cos + torch.cat([-b, a], -1) * sin

            h = F.rms_norm(x, (H,), self.n1, 1e-5)
            q, k, v = (m(h).view(B, S, nh, d).transpose(1, 2) for m in (self.q, self.k, self.v))
            a = F.scaled_dot_product_attention(rope(q), rope(k), v, is_causal=True)
            x = x + self.o(a.transpose(1, 2).reshape(B, S, H))
            h = F.rms_norm(x, (H,), self.n2, 1e-5)
            return x + self.d(F.silu(self.g(h)) * self.u(h))

    def run(mode: str) -> float:
        torch.manual_seed(0)
        emb = nn.Parameter(torch.randn(V, H) * 0.02)
        layers = nn.ModuleList(Layer() for _ in range(L))
        nf = nn.Parameter(torch.ones(H))
        params = [emb, nf, *layers.parameters()]
        with torch.no_grad():
            for p_ in params:
                p_.data = p_.data.to(device=device, dtype=torch.bfloat16)
        master = [p_.detach().float().clone().requires_grad_(True) for p_ in params]
        opt = torch.optim.AdamW(master, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, fused=True)
        inv = 1.0 / (1e4 ** (torch.arange(0, d, 2, device=device, dtype=torch.float32) / d))
        fr = torch.outer(torch.arange(S, device=device, dtype=torch.float32), inv)
        cos, sin = (t.to(torch.bfloat16) for t in (torch.cat([fr, fr], -1).cos(), torch.cat([fr, fr], -1).sin()))
        gen = torch.Generator(device=device).manual_seed(1)
        ids = torch.randint(0, V, (B, S + 1), device=device, generator=gen)
        x_ids, y = ids[:, :S], ids[:, 1:]

        def step():
            for p_ in params:
                p_.grad = None
            x = F.embedding(x_ids, emb)
            for layer in layers:
                x = checkpoint(layer, x, cos, sin, use_reentrant=False) if mode == "full" else layer(x, cos, sin)
            logits = F.rms_norm(x, (H,), nf, 1e-5) @ emb.t()
            F.cross_entropy(logits.float().reshape(-1, V), y.reshape(-1)).backward()
            for m, p_ in zip(master, params):
                m.grad = p_.grad.float()
            torch.nn.utils.clip_grad_norm_(master, 1.0)
            opt.step()
            with torch.no_grad():
                for m, p_ in zip(master, params):
                    p_.copy_(m)

        for _ in range(warmup):
            step()
        torch.cuda.synchronize(device)
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize(device)
        return (time.perf_counter() - t0) / steps

    try:
        t_full = run("full")
        t_none = run("none")
    except Exception as exc:  # context only: never fail the benchmark line for it
        return {"error": f"{type(exc).__name__}: {exc}"}
    return dict(
        workload="the config-3 step in plain PyTorch-ROCm (SDPA, hipBLASLt, F.rms_norm, torch checkpoint, "
                 "fused AdamW on an fp32 master), host-launched, same GPU",
        tokens_per_s=round(B * S / t_full, 1), ms_per_step=round(t_full * 1e3, 3),
        no_checkpoint_tokens_per_s=round(B * S / t_none, 1), steps_timed=steps,
    )


def c5_leg(args, device) -> dict:
    """One ring rank's attention share: rank 3 of 4
    (queries 24576..32767) over the four K/V blocks in ring order 3, 2, 1, 0
    (context_parallel/ring.py:104-250), causal by absolute position, forward
    then backward (P recomputed from the LSE); FLOPs count the visible
    (causally unmasked) scores only, backward 2.5x the forward."""
    import torch

    from nano_megatron_amd import functional as Fn

    s, h, d, nb = 8192, 16, 128, 4
    g = torch.Generator(device=device).manual_seed(5)
    bf = torch.bfloat16
    q = torch.randn(1, s, h, d, device=device, generator=g).to(bf)
    ks = [torch.randn(1, s, h, d, device=device, generator=g).to(bf) for _ in range(nb)]
    vs = [torch.randn(1, s, h, d, device=device, generator=g).to(bf) for _ in range(nb)]
    order = [3, 2, 1, 0]
    kb, vb = [ks[i] for i in order], [vs[i] for i in order]
    offs = tuple(i * s for i in order)
    q_off = 3 * s
    do = torch.randn(1, s, h, d, device=device, generator=g).to(bf)
    dq = torch.empty_like(q)
    dks = [torch.empty_like(k) for k in kb]
    dvs = [torch.empty_like(v) for v in vb]
    o, lse = Fn.attn_fwd_bshd(q, kb, vb, offs, causal=True, q_offset=q_off, scale=None)

    def fwd():
        Fn.attn_fwd_bshd(q, kb, vb, offs, causal=True, q_offset=q_off, scale=None, out=o, lse=lse)

    def bwd():
        Fn.attn_bwd_bshd(q, kb, vb, offs, o, do, lse, dq, dks, dvs, causal=True, q_offset=q_off, scale=None)

    def timed(fn, n):
        for _ in range(max(args.warmup, 1)):
            fn()
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(device)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    full_blocks = 3 * 4 * h * s * s * d          # blocks 2, 1, 0: every score visible
    fwd_flops = full_blocks + 4 * h * s * s * d / 2  # + the diagonal block's causal half
    bwd_flops = 2.5 * fwd_flops
    t_f, t_b = timed(fwd, args.steps), timed(bwd, args.steps)
    tf_f, tf_b = fwd_flops / t_f / 1e9, bwd_flops / t_b / 1e9
    total = (fwd_flops + bwd_flops) / (t_f + t_b) / 1e9
    del q, ks, vs, do, dq, dks, dvs, o, lse
    torch.cuda.empty_cache()
    return dict(
        workload="C5: rank 3 of a 4-way ring, local Q [1, 8192, 16, 128] bf16, K/V blocks visited 3, 2, 1, 0, "
                 "causal by absolute position, forward + backward",
        tflops=round(total, 1), mfma_frac=round(total / BF16_PEAK_TFLOPS, 4), ms=round(t_f + t_b, 3),
        fwd_ms=round(t_f, 3), bwd_ms=round(t_b, 3), fwd_tflops=round(tf_f, 1), bwd_tflops=round(tf_b, 1),
        fwd_gflop=round(fwd_flops / 1e9, 1), bwd_gflop=round(bwd_flops / 1e9, 1),
    )


def run_c4(args, device) -> None:
    leg = c4_leg(args, device, eager=not args.no_eager)
    line = dict(
        metric="train tokens/s, GQA 32q/8kv seq2048 full recompute, 1 MI355X",
        value=leg["tokens_per_s"], unit="tokens/s", n_gpus=1, steps=args.steps,
        warmup=args.warmup, ms_per_step=leg["ms_per_step"], higher_is_better=True,
        scaling="weak", vs_baseline=None, dtype="bf16", data="synthetic",
        config=dict(workload=leg["workload"], global_batch=C4_BATCH, seq_len=C4_SEQ, parallelism="single GPU"),
        **{k: v for k, v in leg.items() if k not in ("workload", "tokens_per_s", "ms_per_step")},
    )
    print(json.dumps(line), flush=True)


def run_c5(args, device) -> None:
    leg = c5_leg(args, device)
    line = dict(
        metric="ring-share attention fwd+bwd TFLOP/s, 8192 queries x 4 K/V blocks, D128, 1 MI355X",
        value=leg["tflops"], unit="TFLOP/s", n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=leg["ms"], higher_is_better=True, scaling="weak", vs_baseline=None,
        dtype="bf16", data="synthetic",
        config=dict(workload=leg["workload"], global_batch=1, seq_len=8192,
                    parallelism="single GPU (one ring rank's share)"),
        roofline=dict(bound="mfma", achieved=leg["tflops"], peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                      frac=leg["mfma_frac"], traffic=None, kernel="attn_fwd + attn_bwd"),
        **{k: v for k, v in leg.items() if k not in ("workload", "tflops", "mfma_frac", "ms")},
    )
    print(json.dumps(line), flush=True)


def main() -> None:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build has no collectives)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X (no HIP device visible)", file=sys.stderr)
        sys.exit(2)
    device = torch.device("cuda", 0)
    import nano_megatron_amd  # noqa: F401  (fails loudly without libnmb.so)
    from nano_megatron_amd import _lib

    _lib.load()
    if args.config == "c4":
        run_c4(args, device)
        return
    if args.config == "c5":
        run_c5(args, device)
        return

    kernels = ceilings = None
    if not args.no_kernels:
        kernels = kernel_rooflines(device, args.kernel if args.only_kernels else None)
        print("kernels: " + json.dumps(kernels), file=sys.stderr, flush=True)
        if not args.kernel:
            ceilings = measured_ceilings(device)
            print("ceilings: " + json.dumps(ceilings), file=sys.stderr, flush=True)
    if args.only_kernels:
        if args.kernel:
            copy_calibration(device)
        return
    full = run_steps("full", args.steps, args.warmup, device, args.metrics_jsonl, graph=not args.host_launch)
    print("full: " + json.dumps(full), file=sys.stderr, flush=True)
    eager = selective = None
    if not args.no_eager:
        eager = run_steps("none", args.steps, args.warmup, device, graph=not args.host_launch)
        print("none: " + json.dumps(eager), file=sys.stderr, flush=True)
        # activation_checkpoint.mode "selective" (attention and MLP sub-blocks
        # checkpointed on their inputs, models/gpt/layer.py:68-89) on the fused block
        selective = run_steps("selective", args.steps, args.warmup, device, graph=not args.host_launch)
        print("selective: " + json.dumps(selective), file=sys.stderr, flush=True)

    c4 = c5 = None
    if not args.no_legs:
        c4 = c4_leg(args, device, eager=not args.no_eager)
        c5 = c5_leg(args, device)
        print("c4: " + json.dumps(c4) + "\nc5: " + json.dumps(c5), file=sys.stderr, flush=True)

    torch_ref = None
    if not args.no_legs and not args.no_torch:
        torch_ref = torch_eager_leg(device)
        print("torch_eager: " + json.dumps(torch_ref), file=sys.stderr, flush=True)

    vendor = None
    if not args.no_legs:
        vendor = vendor_gemm_leg(device)
        print("vendor_gemm: " + json.dumps(vendor), file=sys.stderr, flush=True)

    roofline = None
    if kernels:
        # the kernel with the most time per training step
        dom = max(kernels, key=lambda k: k["us_per_step"])
        if dom["bound"] == "mfma":
            roofline = dict(bound="mfma", achieved=dom["tflops"], peak=BF16_PEAK_TFLOPS, unit="TFLOP/s",
                            frac=dom["mfma_frac"])
        else:
            roofline = dict(bound="hbm", achieved=dom["gbs"], peak=HBM_PEAK_GBS, unit="GB/s",
                            frac=dom["hbm_frac"])
        roofline.update(traffic=measured_traffic(dom["kernel"]), kernel=dom["kernel"],
                        us_per_launch=dom["us"], algorithmic_bytes=dom["bytes"])
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline()
    if kernels and ceilings:
        # each HBM-bound kernel against what a plain device copy reaches on this box
        for k_ in kernels:
            if k_["bound"] == "hbm":
                k_["copy_frac"] = round(k_["gbs"] / ceilings["copy_256mib_gbs"], 3)
    line = dict(
        metric=METRIC,
        value=round(full["tokens_per_s"], 1),
        unit="tokens/s",
        n_gpus=1,
        steps=args.steps,
        warmup=args.warmup,
        ms_per_step=round(full["ms_per_step"], 3),
        # "hip_graph": the step captured once (CapturedTrainStep) and replayed;
        # the same step with every kernel launched from the host, same process:
        launch=full["launch"],
        host_launched_tokens_per_s=round(full["eager_tokens_per_s"], 1),
        host_launched_ms_per_step=round(full["eager_ms_per_step"], 3),
        higher_is_better=True,
        scaling="weak",
        vs_baseline=None,
        dtype="bf16",
        data="synthetic",
        config=dict(
            workload="C3: 310.8M GPT (24L, H1024, 16 heads MHA D64, ffn 2736, vocab 8192 tied) "
                     "training step, full per-layer recompute, bf16 + fp32-master AdamW",
            global_batch=BATCH, seq_len=SEQ, parallelism="single GPU",
        ),
        peak_act_gib_per_layer=round(full["peak_act_gib_per_layer"], 4),
        # one block's saved activation (2-layer minus 1-layer model); the
        # whole-model figure spreads the head's saved state over the layers
        saved_act_mib_per_layer=round(block_saved_mib("full", device), 2),
        act_floor_mib_per_layer=16.0,
        saved_act_mib_whole_model_per_layer=round(full["saved_act_mib_per_layer"], 2),
        model_tflops=round(model_step_flops(C3, BATCH, SEQ, recompute=True) / (full["ms_per_step"] * 1e-3) / 1e12, 1),
        loss=round(full["loss"], 4),
        roofline=roofline,
        cpu_baseline=cpu,
        ceilings=ceilings,
        kernels=kernels,
        c4=c4,
        c5=c5,
        torch_eager=torch_ref,
        vendor_gemm=vendor,
    )
    if eager:
        line["no_checkpoint_tokens_per_s"] = round(eager["tokens_per_s"], 1)
        line["no_checkpoint_saved_act_mib_per_layer"] = round(block_saved_mib("none", device), 2)
        line["recompute_overhead"] = round(full["ms_per_step"] / eager["ms_per_step"] - 1.0, 4)
    if selective:
        line["selective"] = dict(
            selective_ops=["attention", "mlp"],
            tokens_per_s=round(selective["tokens_per_s"], 1),
            ms_per_step=round(selective["ms_per_step"], 3),
            host_launched_tokens_per_s=round(selective["eager_tokens_per_s"], 1),
            recompute_overhead=round(selective["ms_per_step"] / eager["ms_per_step"] - 1.0, 4),
            saved_act_mib_per_layer=round(block_saved_mib("selective", device), 2),
            peak_act_gib_per_layer=round(selective["peak_act_gib_per_layer"], 4),
        )
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
