"""Benchmark: the fusion-template hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]

One step = one causal flash-attention forward at the headline shape
(B=8, H=32, S=4096, D=128, bf16 in, fp32 accumulate, bf16 out + fp32 lse),
inputs resident in HBM. The line also carries the other configurations of the
metric, each timed the same way with HIP events on the launch stream: the
fused row softmax and layernorm ([8192, 4096] fp32, HBM GB/s), split-K GQA
decode, the causal backward, and the next rows (the fused GEMM epilogue, the
map chain, the stencil and a carved gpt2-small forward).

Every output is verified against the float64 oracle before timing
(verify-before-time, as benchmarks/bench_zoo.py:142-150 in the reference).
Rank 0 prints ONE JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA (AMD spec; no sparsity)
PEAK_HBM_GBS = 8000.0  # MI355X HBM3E


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=30)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--settle-ms", type=float, default=300.0,
                   help="untimed back-to-back steps for this long (wall clock) before the warmup, so the timed "
                        "steps run at the part's sustained clock, not its boost after idle (0: none)")
    p.add_argument("--quick", action="store_true", help="skip the secondary configs and the CPU baseline")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--lines", default=None,
                   help="comma-separated subset of the secondary lines to run (profiling one kernel): "
                   + ", ".join(SECONDARY))
    p.add_argument("--gemm-ref", action="store_true", help="also time a plain bf16 GEMM (hipBLASLt) for reference")
    p.add_argument(
        "--copy-probe",
        action="store_true",
        help="also run a plain device copy of known size (the calibration kernel of the FETCH_SIZE / WRITE_SIZE runs)",
    )
    return p.parse_args()


COPY_PROBE_BYTES = 256 << 20  # bytes read (and bytes written) by one calibration copy
PMC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "flash_fwd_m16_c3_pmc.md")


def measured_traffic():
    """HBM bytes per launch of the C3 forward, as the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary states it (a line
    `traffic_bytes_per_launch: N`), or None when no such summary exists."""
    try:
        with open(PMC_SUMMARY) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1].strip()))
    except OSError:
        return None
    return None


def causal_flops(B, H, S, D):
    """Algorithmic FLOPs of causal attention forward: 2 GEMMs (QK^T, PV) of
    2*D FLOP per (query, live key) pair; live pairs = S(S+1)/2 per head."""
    return 4.0 * B * H * D * (S * (S + 1) / 2)


def time_events(fn, iters, warmup=2):
    """Average ms per call, HIP events around `iters` back-to-back calls on
    the current stream (the stream every kernel here launches on). The timed
    calls run under measure.no_compiles: a hipRTC compile inside them (a
    program the warmups did not reach) raises instead of being timed."""
    import torch

    from pdum_dsl_amd.measure import no_compiles

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    with no_compiles("bench timed loop"):
        t0.record()
        for _ in range(iters):
            fn()
        t1.record()
        torch.cuda.synchronize()
    return t0.elapsed_time(t1) / iters


def main():
    a = _args()
    if a.gpus != 1:
        print(
            f"bench.py: this build measures one GPU only (asked for {a.gpus}); every benchmark config fits one "
            "MI355X and the hot path has no cross-GPU exchange to measure",
            file=sys.stderr,
        )
        sys.exit(2)
    import torch

    from oracle import closed_forms as cf
    from pdum_dsl_amd import kernels as K

    dev = torch.device("cuda:0")
    h = lambda t: t.float().cpu().numpy().astype(np.float64)  # noqa: E731

    # ---------------- C3: causal flash forward (the step) ----------------
    B, H, S, D = 8, 32, 4096, 128
    g = torch.Generator(device=dev).manual_seed(3)
    q, k, v = (torch.randn((B, H, S, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16) for _ in range(3))
    scale = 1.0 / math.sqrt(D)
    o = torch.empty_like(q)

    def step():
        return K.flash_fwd(q, k, v, scale=scale, band=K.CAUSAL, out=o)

    res = step()
    torch.cuda.synchronize()
    verify = []
    for bh in ((0, 0), (B - 1, H - 1)):  # verify before timing
        wo, _, _, wl = cf.attention(h(q[bh]), h(k[bh]), h(v[bh]), scale=scale, band=(None, 0))
        err = float(np.abs(h(res.o[bh]) - wo).max())
        lerr = float(np.abs(h(res.lse[bh]) - wl).max())
        lrel = float((np.abs(h(res.lse[bh]) - wl) / np.maximum(1.0, np.abs(wl))).max())
        assert err <= 2e-2 * max(1.0, float(np.abs(wo).max())) and lrel <= 1e-5, \
            f"flash fwd parity failed at {bh}: out {err}, lse {lerr} ({lrel:.2e} relative)"
        verify.append({"instance": list(bh), "max_abs_err_out": err, "max_abs_err_lse": lerr})

    if a.copy_probe:  # a plain copy of known size, for scaling the HBM byte counters
        src = torch.empty(COPY_PROBE_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # settle: after idle the part first runs above its sustained clock, then
    # its power management pulls the clock down under back-to-back load (a
    # dip of up to ~30% per step before it levels off). Back-to-back steps
    # for a fixed wall time (a sync every 8 keeps the wall clock honest and
    # the queue full), then the W warmup steps, then exactly K timed steps:
    # the timed steps measure the sustained rate.
    n_settle, t_settle = 0, time.perf_counter()
    while time.perf_counter() - t_settle < a.settle_ms / 1e3:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
        n_settle += 8
    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    from pdum_dsl_amd.measure import no_compiles

    wall0 = time.perf_counter()
    with no_compiles("bench headline loop"):
        e0.record()
        for _ in range(a.steps):
            step()
        e1.record()
        torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = e0.elapsed_time(e1) / a.steps
    flops = causal_flops(B, H, S, D)
    tflops = flops / (ms * 1e-3) / 1e12

    line = {
        "metric": "flash-attn fwd TFLOP/s (% MFMA peak) + fused softmax HBM GB/s, 1xMI355X",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "settle": {"steps": n_settle, "ms": a.settle_ms,
                   "why": "untimed back-to-back steps before the warmup: the timed steps run at the sustained clock"},
        "ms_per_step": round(ms, 4),
        "wall_s_timed": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1))",
        "config": {
            "workload": "C3 causal flash-attention forward (fusion template 'flash'), B=8 H=32 S=4096 D=128, "
            "bf16 in / fp32 accumulate / bf16 out + fp32 lse",
            "batch": B,
            "heads": H,
            "seq_len": S,
            "head_dim": D,
            "parallelism": "single GPU",
        },
        "roofline": {
            "kernel": "flash_fwd_m16<bf16,128>",
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
            "traffic": measured_traffic(),
            "algorithmic_flop_per_launch": flops,
        },
        "verify": verify,
    }

    if not a.quick:
        line["secondary"] = secondary(torch, K, cf, h, dev, None if a.lines is None else set(a.lines.split(",")))
    if a.gemm_ref:
        line["gemm_reference"] = gemm_reference(torch, dev)
    if not a.quick and not a.no_cpu:
        line["cpu_baseline"] = cpu_baseline(cf)
    print(json.dumps(line), flush=True)


SECONDARY = ("attention_c1", "row_softmax", "layernorm", "decode", "flash_bwd", "contraction_epilogue", "map_chain",
             "stencil", "carved_plan", "carved_grad")


def secondary(torch, K, cf, h, dev, sel=None):
    """The secondary lines (all of SECONDARY, or the names in ``sel``), each
    on inputs from its own seeded generator, each verified before it is
    timed; a line that fails reports its error instead of a number."""
    out = {}
    on = lambda n: sel is None or n in sel  # noqa: E731
    gen = lambda seed: torch.Generator(device=dev).manual_seed(seed)  # noqa: E731
    lines = [
        (("attention_c1",), lambda: _c1_line(torch, K, cf, h, dev, gen(1))),
        (("row_softmax", "layernorm"), lambda: _c2_lines(torch, K, cf, h, dev, gen(2), on)),
        (("decode",), lambda: _c4_line(torch, K, cf, h, dev, gen(4))),
        (("flash_bwd",), lambda: _c5_line(torch, K, cf, h, dev, gen(5))),
        (("contraction_epilogue",), lambda: _contraction_line(torch, K, dev, gen(6))),
        (("map_chain",), lambda: _map_chain_line(torch, K, dev, gen(7))),
        (("stencil",), lambda: _stencil_line(torch, K, dev, gen(8))),
        (("carved_plan",), lambda: _carved_plan_line(torch)),
        (("carved_grad",), lambda: _carved_grad_line(torch)),
    ]
    for names, fn in lines:
        if not any(on(n) for n in names):
            continue
        try:
            res = fn()
            out.update(res if len(names) > 1 else {names[0]: res})
        except Exception as exc:  # reported in the line, never hidden
            out.update({n: {"error": str(exc)} for n in names if on(n)})
    return out


def _c1_line(torch, K, cf, h, dev, g):
    """C1: single-head non-causal attention, S=256 D=64 fp32."""
    T1, D1 = 256, 64
    q1, k1, v1 = (torch.randn((1, 1, T1, D1), generator=g, device=dev, dtype=torch.float32) for _ in range(3))
    r1 = K.flash_fwd(q1, k1, v1, scale=D1**-0.5)
    torch.cuda.synchronize()
    wo = cf.attention(h(q1[0, 0]), h(k1[0, 0]), h(v1[0, 0]), scale=D1**-0.5)[0]
    err = float(np.abs(h(r1.o[0, 0]) - wo).max())
    assert err <= 1e-5 * max(1.0, float(np.abs(wo).max())), f"C1 parity failed: {err}"
    ms_eager = time_events(lambda: K.flash_fwd(q1, k1, v1, scale=D1**-0.5, out=r1.o), 200)
    # one call is a single small launch, so the wrapper's loop times its host work; the
    # prepared call (geometry and pointers bound once) is the launch alone
    call = K.flash_fwd_prepared(q1, k1, v1, scale=D1**-0.5, out=r1.o)
    r1.o.zero_()
    call()
    torch.cuda.synchronize()
    perr = float(np.abs(h(r1.o[0, 0]) - wo).max())
    assert perr == err, f"C1 prepared call differs from the wrapper's: {perr} vs {err}"
    ms = time_events(call, 200)
    fl = 4.0 * D1 * T1 * T1
    return {
        "config": "C1 B=1 H=1 S=256 D=64 non-causal fp32", "ms": round(ms, 5), "TFLOP/s": round(fl / ms / 1e9, 3),
        "algorithmic_flop": fl, "max_abs_err": err, "ms_wrapper_call": round(ms_eager, 5),
        "note": "one head: 4 query workgroups on a 256-CU chip, latency-bound by construction; ms times the "
                "prepared call (kernels.flash_fwd_prepared), ms_wrapper_call the per-call Python wrapper",
    }


def _c2_lines(torch, K, cf, h, dev, g, on):
    """C2: row softmax and layernorm over [8192, 4096] fp32."""
    out = {}
    R, C = 8192, 4096
    x = torch.randn((R, C), generator=g, device=dev, dtype=torch.float32)
    gamma = (1 + 0.1 * torch.randn((C,), generator=g, device=dev)).float()
    beta = (0.1 * torch.randn((C,), generator=g, device=dev)).float()
    y = torch.empty_like(x)
    rows = [0, R // 2, R - 1]
    if on("row_softmax"):
        K.row_softmax(x, out=y)
        torch.cuda.synchronize()
        err = float(np.abs(h(y[rows]) - cf.np_softmax(h(x[rows]), axis=1)).max())
        assert err < 1e-6, f"softmax parity failed: {err}"
        ms = time_events(lambda: K.row_softmax(x, out=y), 50)
        nbytes = 2 * R * C * 4
        out["row_softmax"] = {
            "config": "C2a [8192,4096] fp32", "ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
            "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4), "bytes": nbytes, "max_abs_err": err,
        }
    if on("layernorm"):
        K.layernorm(x, gamma, beta, 1e-5, out=y)
        torch.cuda.synchronize()
        want = cf.np_layernorm(h(x[rows]), h(gamma), h(beta), 1e-5)
        err = float(np.abs(h(y[rows]) - want).max())
        assert err < 1e-4, f"layernorm parity failed: {err}"
        ms = time_events(lambda: K.layernorm(x, gamma, beta, 1e-5, out=y), 50)
        nbytes = 2 * R * C * 4 + 2 * C * 4
        out["layernorm"] = {
            "config": "C2b [8192,4096] fp32 + gamma/beta", "ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
            "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4), "bytes": nbytes, "max_abs_err": err,
        }
    return out


def _c4_line(torch, K, cf, h, dev, g):
    """C4: grouped-query decode, split-K."""
    Bd, Hq, Hkv, Sk, D = 64, 32, 8, 8192, 128
    qd = torch.randn((Bd, Hq, 1, D), generator=g, device=dev).to(torch.bfloat16)
    kc = torch.randn((Bd, Hkv, Sk, D), generator=g, device=dev).to(torch.bfloat16)
    vc = torch.randn((Bd, Hkv, Sk, D), generator=g, device=dev).to(torch.bfloat16)
    nsplit = K.pick_decode_splits(Bd * Hkv, Sk)
    ws = torch.empty(Bd * Hq * nsplit * (2 + D), dtype=torch.float32, device=dev)
    od, lse = K.attn_decode(qd, kc, vc, nsplit=nsplit, workspace=ws)
    torch.cuda.synchronize()
    errs = []
    for b, hq in ((0, 0), (Bd - 1, Hq - 1)):
        wo, _, _, wl = cf.attention(h(qd[b, hq]), h(kc[b, hq // 4]), h(vc[b, hq // 4]), scale=D**-0.5)
        errs.append(float(np.abs(h(od[b, hq]) - wo).max()))
    assert max(errs) < 2e-2, f"decode parity failed: {errs}"
    ms = time_events(lambda: K.attn_decode(qd, kc, vc, nsplit=nsplit, workspace=ws), 30)
    nbytes = 2 * Bd * Hkv * Sk * D * 2
    return {
        "config": "C4 B=64 Hq=32 Hkv=8 Sk=8192 D=128 bf16", "nsplit": nsplit, "ms": round(ms, 5),
        "GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
        "kv_bytes": nbytes, "max_abs_err": max(errs),
    }


def _c5_line(torch, K, cf, h, dev, g):
    """C5: causal backward, B=4 H=16 S=2048 D=64 bf16."""
    Bb, Hb, Sb, Db = 4, 16, 2048, 64
    qb, kb, vb, dob = (torch.randn((Bb, Hb, Sb, Db), generator=g, device=dev).to(torch.bfloat16) for _ in range(4))
    fw = K.flash_fwd(qb, kb, vb, band=K.CAUSAL)
    dq, dk, dv = K.flash_bwd(qb, kb, vb, fw.o, dob, fw.lse, band=K.CAUSAL)
    torch.cuda.synchronize()
    wq, wk, wv = cf.attention_bwd(h(qb[0, 0]), h(kb[0, 0]), h(vb[0, 0]), h(dob[0, 0]), scale=Db**-0.5,
                                  band=(None, 0))
    errs = {
        nm: float(np.abs(h(t[0, 0]) - w).max() / max(1.0, np.abs(w).max()))
        for nm, t, w in (("dq", dq, wq), ("dk", dk, wk), ("dv", dv, wv))
    }
    assert max(errs.values()) < 2e-2, f"backward parity failed: {errs}"
    ms = time_events(lambda: K.flash_bwd(qb, kb, vb, fw.o, dob, fw.lse, band=K.CAUSAL), 20)
    fl = 2.5 * causal_flops(Bb, Hb, Sb, Db)
    return {
        "config": "C5 causal bwd B=4 H=16 S=2048 D=64 bf16", "ms": round(ms, 5),
        "TFLOP/s": round(fl / ms / 1e9, 2), "frac_mfma": round(fl / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
        "algorithmic_flop": fl, "rel_err": errs,
    }


def _stencil_line(torch, K, dev, g):
    """The stencil template's 5-point update u + alpha * laplacian(u) over the
    interior of an 8194 x 8194 fp32 halo, planned by plan_region (template
    "stencil") and run as one elementwise program whose five neighbor reads
    are offset views of u (reuse through L1 / L2)."""
    from pdum_dsl_amd import ewprog
    from pdum_dsl_amd.tl import fusion, zoo

    MI = NI = 8192
    s = zoo.stencil_tile(MI=MI, NI=NI, alpha=0.1, seed=3)
    (grp,) = fusion.plan_region(s.naive).groups
    y = s.naive.body[-1].args[0]
    p = s.naive.params[0]
    low = ewprog.lower(y, y.type.dims, {id(p): p}, allow_views=True)
    u = torch.randn((MI + 2, NI + 2), generator=g, device=dev)
    out = torch.empty((MI, NI), device=dev)
    views = [low.operand_view(j, {"x": u.stride(0), "y": u.stride(1)}) for j in range(len(low.operands))]
    prog = low.program(out.stride(), [st for st, _o in views])
    ops = [u.reshape(-1)[o:] for _st, o in views]
    K.map_chain(prog, ops, out)
    torch.cuda.synchronize()
    rows = [0, MI // 2, MI - 1]
    uc = u.double().cpu().numpy()
    want = s.oracle([uc])[rows]
    err = float(np.abs(out[rows].double().cpu().numpy() - want).max())
    assert err < 1e-5 * max(1.0, float(np.abs(want).max())), f"stencil parity failed: {err}"
    ms = time_events(lambda: K.map_chain(prog, ops, out), 30)
    nbytes = ((MI + 2) * (NI + 2) + MI * NI) * 4
    return {
        "config": f"u + 0.1 * (5-point laplacian) over [{MI}, {NI}] fp32 (halo [{MI + 2}, {NI + 2}]); template "
                  f"{grp.template} ({grp.certificate.verdict}), {len(low.operands)} shifted views, "
                  f"{len(low.insns)} instructions",
        "ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
        "bytes": nbytes, "max_abs_err": err,
    }


def _gpt2_torch(torch, W, cfg):
    """The same forward with torch's own kernels (hipBLASLt matmuls, separate
    elementwise ops): the comparator for the carved plan. Right operands of
    every batched product are contiguous."""
    F = torch.nn.functional
    T, D, H, Kh = cfg.t, cfg.d, cfg.nh, cfg.hk
    h = W["wte"][W["ids"]] + W["wpe"]
    mask = torch.ones((T, T), dtype=torch.bool, device=h.device).tril()
    for i in range(cfg.layers):
        p = f"h.{i}."
        a = F.layer_norm(h, (D,), W[p + "attn.ln1g"], W[p + "attn.ln1b"], eps=cfg.eps)
        q = (a @ W[p + "attn.wq2"]).view(T, H, Kh).transpose(0, 1) * (Kh ** -0.5)
        k = (a @ W[p + "attn.wk2"]).view(T, H, Kh).permute(1, 2, 0).contiguous()
        v = (a @ W[p + "attn.wv2"]).view(T, H, Kh).transpose(0, 1).contiguous()
        sc = torch.matmul(q, k).masked_fill(~mask, -1e9)
        cx = torch.matmul(torch.softmax(sc, dim=-1), v).transpose(0, 1).reshape(T, H * Kh)
        h = h + cx @ W[p + "attn.wo2"]
        a2 = F.layer_norm(h, (D,), W[p + "mlp.ln2g"], W[p + "mlp.ln2b"], eps=cfg.eps)
        u = F.gelu(a2 @ W[p + "mlp.w1"] + W[p + "mlp.b1"], approximate="tanh")
        h = h + u @ W[p + "mlp.w2"] + W[p + "mlp.b2"]
    hf = F.layer_norm(h, (D,), W["lnfg"], W["lnfb"], eps=cfg.eps)
    return hf @ W["wteT"]


def _carved_plan_line(torch):
    """gpt2-small's shape (12 layers, t=1024, d=768, 12 heads of 64, mlp 3072,
    vocab 50257), random weights, bf16: planned by plan_model (the
    anchor-and-absorb partition) and run by the device executor, every
    boundary in HBM, the pass captured as one HIP graph (``ms``; the
    per-kernel launched pass is ``ms_eager_launches``; each layer's softmax
    and PV carves run as one flash launch, and ``ms_without_attention_chains``
    times the same plan with every carve launched apart). Checked against the
    same forward in fp32 on the same bf16 weights; timed beside torch's own
    bf16 forward (eager)."""
    import time as _time

    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.partition import plan_model

    cfg = zoo.GPT2Config(t=1024, d=768, nh=12, hk=64, m=3072, layers=12, v=50257)
    t0 = _time.perf_counter()
    m = zoo.gpt2(cfg, seed=7)
    plan = plan_model(m.region)
    ex = PlanExecutor(plan, m.region, "bf16")
    plan_s = _time.perf_counter() - t0
    ex.bind(m.values())
    y = m.region.body[-1].args[0]
    got = ex.run()
    torch.cuda.synchronize()
    W = {m.names[id(p)]: t for p, t in zip(m.region.params, (ex.bound[id(p)] for p in m.region.params))}
    for i in range(cfg.layers):
        p = f"h.{i}."
        for nm in ("wq", "wk", "wv"):
            W[p + f"attn.{nm}2"] = W[p + f"attn.{nm}"].reshape(cfg.d, cfg.nh * cfg.hk)
        W[p + "attn.wo2"] = W[p + "attn.wo"].reshape(cfg.nh * cfg.hk, cfg.d)
    W["wteT"] = W["wte"].t().contiguous()
    W32 = {k: (v.float() if v.is_floating_point() else v) for k, v in W.items()}
    want = _gpt2_torch(torch, W32, cfg)
    gotv = got.float().permute([y.type.names.index(n) for n in m.order])
    scale = float(want.abs().max())
    err = float((gotv - want).abs().max())
    assert err < 5e-2 * scale, f"carved-plan parity failed: {err} vs scale {scale}"
    del W32, want, gotv
    eager = ex.run().clone()
    ms_eager = time_events(ex.run, 10)
    ex.capture()
    replayed = ex.replay()
    torch.cuda.synchronize()
    assert torch.equal(replayed, eager), "the captured plan's replay differs from the eager pass"
    ms = time_events(lambda: ex.replay(check=False), 20)
    ms_torch = time_events(lambda: _gpt2_torch(torch, W, cfg), 10)
    # the same plan with every carve its own launch (scores, softmax and PV apart)
    ex2 = PlanExecutor(plan, m.region, "bf16", fuse_attention=False)
    ex2.bind(m.values())
    ex2.capture()
    ms_unfused = time_events(lambda: ex2.replay(check=False), 20)
    del ex2
    T, D, M, V, L_ = cfg.t, cfg.d, cfg.m, cfg.v, cfg.layers
    fl = 2.0 * T * (L_ * (4 * D * D + 2 * D * M) + D * V) + L_ * 4.0 * T * T * D
    by = {}
    for c in plan.carves:
        by[c.group.template] = by.get(c.group.template, 0) + 1
    return {
        "config": "gpt2-small shape, 12 layers, t=1024 tokens, d=768, 12x64 heads, mlp 3072, vocab 50257, bf16 "
                  "storage / fp32 accumulate; random weights",
        "carves": by, "device_steps": len(ex.steps) + sum(len(n.steps) for n in ex.nested),
        "attention_chains": sum(st.kind == "flash-chain" for st in ex.steps),
        "ms_without_attention_chains": round(ms_unfused, 4),
        "plan_s": round(plan_s, 2), "ms": round(ms, 4), "ms_eager_launches": round(ms_eager, 4),
        "tokens_per_s": round(T / ms * 1e3, 1),
        "TFLOP/s": round(fl / ms / 1e9, 1), "algorithmic_flop": fl,
        "torch_eager_ms": round(ms_torch, 4), "max_abs_err_vs_f32": err, "logit_scale": scale,
    }


def _carved_grad_line(torch, dtype="f32"):
    """A gpt2-small training step's compute: the joint of the forward and the
    gradients of every weight, the embedding tables included (autodiff.grad
    of the logits, seeded by a random cotangent; wte's gradient is the
    scatter-add of the embedding's cotangent plus the tied head's product),
    planned by plan_model and run by the device executor as one HIP graph. fp32 storage: the carved backward
    rounds every boundary to the storage type, and in bf16 the layernorm and
    softmax backward carves cancel (layer 0's gradients drift far from fp32
    over 12 layers). The contractions run on the bf16 matrix cores with the
    fp32 operands split into bf16 planes: six products per term (fp32 grade,
    ``ms``), and, timed beside it, three (about 2^-16 of each product,
    ``ms_bf16x3``).
    Checked against torch fp32 autograd of the same forward on the same
    weights (four gradients, wte among them), and timed beside torch's
    forward + backward (eager autograd, fp32, the same weights)."""
    import time as _time

    from pdum_dsl_amd.executor import PlanExecutor
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names
    from pdum_dsl_amd.tl.partition import plan_model

    cfg = zoo.GPT2Config(t=1024, d=768, nh=12, hk=64, m=3072, layers=12, v=50257)
    t0 = _time.perf_counter()
    m = zoo.gpt2(cfg, seed=7)
    pn = tuple(m.names[id(p)] for p in m.region.params)
    wrt = tuple(n for n in pn if n != "ids")
    rg = grad(m.region, "logits", seed="dlogits", wrt=wrt, names=region_names(m.region, pn, ("logits",)))
    plan = plan_model(rg.region)
    ex = PlanExecutor(plan, rg.region, dtype, f32_contract="bf16x6")
    plan_s = _time.perf_counter() - t0
    seed_t = rg.region.params[-1].type
    dl = np.random.default_rng(9).standard_normal(tuple(seed_t.shape)) * 1e-2
    ex.bind(m.values() + [dl])
    outs = ex.run()
    torch.cuda.synchronize()
    ex.capture()
    ms = time_events(lambda: ex.replay(check=False), 10)
    # torch: the same forward with autograd on the same fp32 weights
    W = {m.names[id(p)]: ex.bound[id(p)] for p in m.region.params}
    W32 = {}
    for k_, v_ in W.items():
        W32[k_] = v_.float().clone().requires_grad_(k_ in wrt) if v_.is_floating_point() else v_
    for i in range(cfg.layers):
        p = f"h.{i}."
        for nm in ("wq", "wk", "wv"):
            W32[p + f"attn.{nm}2"] = W32[p + f"attn.{nm}"].reshape(cfg.d, cfg.nh * cfg.hk)
        W32[p + "attn.wo2"] = W32[p + "attn.wo"].reshape(cfg.nh * cfg.hk, cfg.d)
    W32["wteT"] = W32["wte"].t().contiguous()
    dlt = torch.as_tensor(dl, dtype=torch.float32, device="cuda").to(ex.bound[id(rg.region.params[-1])].dtype).float()
    dlt = dlt.permute([seed_t.names.index(n) for n in m.order])
    _gpt2_torch(torch, W32, cfg).backward(dlt)

    def rel_errs(outs_):
        errs_ = {}
        by = dict(zip(rg.outputs, outs_))
        for nm in ("h.0.mlp.w1", "h.11.mlp.w2", "lnfg", "wte"):
            node = rg.nodes[rg.grads[nm]]
            pt = next(p for p in m.region.params if m.names[id(p)] == nm).type
            got = by[rg.grads[nm]].float().permute([node.type.names.index(d) for d in pt.names])
            want = W32[nm].grad
            errs_[nm] = float((got - want).abs().max() / want.abs().max())
        return errs_

    errs = rel_errs(outs)
    assert max(errs.values()) < (1e-3 if dtype == "f32" else 0.25), f"carved-gradient parity failed: {errs}"
    ex.release_graph()
    ex_b = PlanExecutor(plan, rg.region, dtype, f32_contract="bf16x3")
    ex_b.bind(m.values() + [dl])
    errs_b = rel_errs(ex_b.run())
    torch.cuda.synchronize()
    assert max(errs_b.values()) < 5e-3, f"carved-gradient parity (bf16x3 contractions) failed: {errs_b}"
    ex_b.capture()
    ms_b = time_events(lambda: ex_b.replay(check=False), 10)
    ex_b.release_graph()
    del W32, ex_b
    Wt = {}
    for k_, v_ in W.items():
        Wt[k_] = v_.clone().requires_grad_(k_ in wrt) if v_.is_floating_point() else v_

    def torch_step():
        for i in range(cfg.layers):
            p = f"h.{i}."
            for nm in ("wq", "wk", "wv"):
                Wt[p + f"attn.{nm}2"] = Wt[p + f"attn.{nm}"].reshape(cfg.d, cfg.nh * cfg.hk)
            Wt[p + "attn.wo2"] = Wt[p + "attn.wo"].reshape(cfg.nh * cfg.hk, cfg.d)
        Wt["wteT"] = Wt["wte"].t().contiguous()
        torch.autograd.grad(_gpt2_torch(torch, Wt, cfg), [Wt[n] for n in wrt], dlt)

    ms_torch = time_events(torch_step, 5)
    by_t = {}
    for c in plan.carves:
        by_t[c.group.template] = by_t.get(c.group.template, 0) + 1
    return {
        "config": "gpt2-small shape (as the carved_plan line), forward + gradients of every weight (the "
                  f"embedding tables included), {dtype} storage / fp32 accumulate; random weights and cotangent",
        "carves": by_t, "device_steps": len(ex.steps), "plan_s": round(plan_s, 2), "ms": round(ms, 4),
        "tokens_per_s": round(cfg.t / ms * 1e3, 1), "ms_bf16x3": round(ms_b, 4),
        "torch_eager_fwd_bwd_ms": round(ms_torch, 4), "torch_dtype": "f32",
        "max_rel_err_vs_torch_f32": errs, "max_rel_err_vs_torch_f32_bf16x3": errs_b,
    }


def _contraction_line(torch, K, dev, g):
    """The planner's contraction-epilogue kernel for the MLP up-projection
    (8192 tokens x 768 -> 3072, gpt2's c_fc width) bound to pdh_contract: the
    epilogue program (bias + tanh-gelu) runs on the accumulators."""
    from pdum_dsl_amd import ewprog
    from pdum_dsl_amd.hip_tile import recognize_contraction
    from pdum_dsl_amd.tl import fusion, zoo
    from pdum_dsl_amd.tl.ir import Dim

    T, D, F = 8192, 768, 3072
    subj = zoo.linear_gelu(T=T, D=D, F=F)
    (grp,) = fusion.plan_region(subj.region).groups
    cb = recognize_contraction(grp.kernel)
    lat = (Dim("_unit", 0, 1), cb["fold"].type.dim("t"), cb["fold"].type.dim("f"))
    low = ewprog.lower(grp.kernel.body[-1].args[0], lat, {id(p): p for p in grp.kernel.params}, acc=cb["fold"])
    x = torch.randn((1, T, D), generator=g, device=dev).to(torch.bfloat16)
    wt = (torch.randn((1, F, D), generator=g, device=dev) * D**-0.5).to(torch.bfloat16)  # w^T: k-contiguous rows
    bias = (0.1 * torch.randn((F,), generator=g, device=dev)).to(torch.bfloat16)
    y = torch.empty((1, T, F), device=dev, dtype=torch.bfloat16)
    prog = low.program(y.stride(), [ewprog.strides_over(bias.stride(), ("f",), lat)])
    K.contract(x, wt, D, prog, [bias], y)
    torch.cuda.synchronize()
    rows = [0, T // 2, T - 1]
    xs, ws, bs = (t.float().cpu().numpy().astype(np.float64) for t in (x[0, rows], wt[0], bias))
    want = subj.oracle([xs, ws.T, bs])
    err = float(np.abs(y[0, rows].float().cpu().numpy() - want).max())
    assert err < 2e-2 * max(1.0, float(np.abs(want).max())), f"contraction-epilogue parity failed: {err}"
    ms = time_events(lambda: K.contract(x, wt, D, prog, [bias], y), 20)
    fl = 2.0 * T * D * F
    return {
        "config": "gelu_tanh(x @ w + b): x [8192, 768] bf16, w [768, 3072], fp32 accumulate; template "
                  f"{grp.template} ({grp.certificate.verdict}), epilogue {len(low.insns)} instructions",
        "ms": round(ms, 5), "TFLOP/s": round(fl / ms / 1e9, 2), "frac_mfma": round(fl / ms / 1e9 / PEAK_BF16_TFLOPS, 4),
        "algorithmic_flop": fl, "max_abs_err": err,
    }


def _map_chain_line(torch, K, dev, g):
    from pdum_dsl_amd import ewprog
    from pdum_dsl_amd.tl import fusion, zoo

    I, J = 8192, 4096
    subj = zoo.masked_activation(I=I, J=J)
    (grp,) = fusion.plan_region(subj.region).groups
    y0 = grp.kernel.body[-1].args[0]
    low = ewprog.lower(y0, y0.type.dims, {id(p): p for p in grp.kernel.params})
    x = torch.randn((I, J), generator=g, device=dev)
    sv = torch.randn((J,), generator=g, device=dev)
    y = torch.empty_like(x)
    prog = low.program(y.stride(), [list(x.stride()), [0, 1]])
    K.map_chain(prog, [x, sv], y)
    torch.cuda.synchronize()
    rows = [0, I // 2, I - 1]
    full = subj.oracle([x.cpu().numpy().astype(np.float64), sv.cpu().numpy().astype(np.float64)])
    err = float(np.abs(y[rows].cpu().numpy() - full[rows]).max())
    assert err < 1e-5, f"map-chain parity failed: {err}"
    ms = time_events(lambda: K.map_chain(prog, [x, sv], y), 30)
    nbytes = 2 * I * J * 4 + J * 4
    return {
        "config": f"where(j > i, tanh(x s_j) + exp(-|x|), 0) over [8192, 4096] fp32; {len(low.insns)} instructions",
        "ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1), "frac_hbm": round(nbytes / ms / 1e6 / PEAK_HBM_GBS, 4),
        "bytes": nbytes, "max_abs_err": err,
    }


def host_facts() -> dict:
    """The host the CPU rows ran on: CPU model, os.cpu_count() and the
    threads torch's CPU kernels use (the region interpreter's parallelism)."""
    import torch

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "torch_threads": int(torch.get_num_threads())}


def median_laps(fn, budget_s: float, min_laps: int = 3, warmup: int = 1):
    """(median seconds per call, laps): ``warmup`` untimed calls, then timed
    calls until both ``min_laps`` and ``budget_s`` are reached (the
    reference's bench_zoo.py:130-150 discipline: verify first, warm, median)."""
    for _ in range(warmup):
        fn()
    laps, t_end = [], time.perf_counter() + budget_s
    while len(laps) < min_laps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        fn()
        laps.append(time.perf_counter() - t0)
    laps.sort()
    return laps[len(laps) // 2], len(laps)


def _tile_program(region):
    """The kernel the fusion planner generates for a one-template region."""
    from pdum_dsl_amd.tl import fusion

    (g,) = fusion.plan_region(region).groups
    return g


def cpu_rows(cf, host) -> list:
    """The reference's CPU evaluator on C1 and C2 whole: the generated tile
    programs run by the float64 region interpreter (oracle.region_eval, the
    torch-CPU evaluator restated), each verified against its closed form
    before it is timed, each reported in its GPU row's own unit."""
    from oracle import region_eval as rev
    from pdum_dsl_amd.tl import zoo

    rows = []
    # C1: single-head non-causal attention, S=256 D=64, the flash tile program
    T, D = 256, 64
    subj = zoo.attention(T=T, S=T, E=D, OD=D, mask="all", seed=3, scale=D**-0.5)
    g = _tile_program(subj.region)
    vals = [rev.value(f.arr, p.type) for f, p in zip(subj.inputs, g.kernel.params)]
    want = cf.attention(*subj.numpy_inputs(), scale=1.0)[0]
    err = float(np.abs(rev.evaluate(g.kernel, vals).numpy(("t", "o")) - want).max())
    assert err < 1e-9, f"C1 CPU row disagrees with the closed form: {err}"
    sec, laps = median_laps(lambda: rev.evaluate(g.kernel, vals), 3.0)
    fl = 4.0 * D * T * T
    rows.append({"config": "C1 B=1 H=1 S=256 D=64 non-causal, whole", "template": g.template,
                 "si": dict(g.params).get("si"), "value": round(fl / sec / 1e12, 8), "unit": "TFLOP/s",
                 "ms": round(sec * 1e3, 3), "laps": laps, "max_abs_err": err, **host})
    # C2a / C2b: row softmax and layernorm over [8192, 4096], whole
    R, C = 8192, 4096
    for name, subj, nbytes in (
        ("C2a row softmax [8192,4096], whole", zoo.row_softmax(rows=R, cols=C, seed=1), 2 * R * C * 4),
        ("C2b layernorm [8192,4096] + gamma/beta, whole", zoo.layernorm(rows=R, feat=C, seed=1),
         2 * R * C * 4 + 2 * C * 4),
    ):
        g = _tile_program(subj.region)
        vals = [rev.value(f.arr, p.type) for f, p in zip(subj.inputs, g.kernel.params)]
        y = g.kernel.body[-1].args[0]
        got = rev.evaluate(g.kernel, vals).numpy(y.type.names)
        want = subj.oracle(subj.numpy_inputs())
        err = float(np.abs(got - want).max())
        assert err < 1e-9, f"{name}: CPU row disagrees with the closed form: {err}"
        del got
        sec, laps = median_laps(lambda: rev.evaluate(g.kernel, vals), 6.0)
        rows.append({"config": name, "template": g.template, "value": round(nbytes / sec / 1e9, 3), "unit": "GB/s",
                     "ms": round(sec * 1e3, 1), "laps": laps, "bytes": nbytes, "max_abs_err": err, **host})
    rows.append(cpu_row_c4(cf, host))
    rows.append(cpu_row_c5(cf, host))
    return rows


def cpu_row_c4(cf, host) -> dict:
    """C4 (grouped-query decode, B=64, 32 query / 8 KV heads, Sk=8192, D=128):
    the flash tile program on one (b, query head) instance — one query row
    against its KV head's 8192 keys — verified, then timed as the median of
    laps. The CPU evaluator serves each query head on its own, so the full
    config is 64 x 32 such instances; the row reports GB/s of the GPU row's
    K/V bytes (each KV head's bf16 K and V once: 2 GiB) over that
    extrapolated time."""
    from oracle import region_eval as rev
    from pdum_dsl_amd.tl import zoo

    B, Hq, Hkv, S, D = 64, 32, 8, 8192, 128
    subj = zoo.attention(T=1, S=S, E=D, OD=D, mask="all", seed=4, scale=D**-0.5)
    g = _tile_program(subj.region)
    vals = [rev.value(f.arr, p.type) for f, p in zip(subj.inputs, g.kernel.params)]
    want = cf.attention(*subj.numpy_inputs(), scale=1.0)[0]
    err = float(np.abs(rev.evaluate(g.kernel, vals).numpy(("t", "o")) - want).max())
    assert err < 1e-9, f"C4 CPU row disagrees with the closed form: {err}"
    sec, laps = median_laps(lambda: rev.evaluate(g.kernel, vals), 3.0)
    n_inst = B * Hq
    full_s = sec * n_inst
    kv_bytes = 2 * B * Hkv * S * D * 2
    return {"config": "C4 B=64 Hq=32 Hkv=8 Sk=8192 D=128: one (b, query head) instance, extrapolated",
            "template": g.template, "si": dict(g.params).get("si"), "value": round(kv_bytes / full_s / 1e9, 4),
            "unit": "GB/s", "ms_one_instance": round(sec * 1e3, 2), "laps": laps, "max_abs_err": err,
            "extrapolated_full_ms": round(full_s * 1e3, 1),
            "extrapolation": f"{n_inst} query-head instances x the one-instance time (the evaluator re-reads a KV "
                             f"head for each of its {Hq // Hkv} query heads)", **host}


def cpu_row_c5(cf, host) -> dict:
    """C5 (causal backward, B=4 H=16 S=2048 D=64): grad's joint region of the
    naive attention twin (the reference's autodiff output, run as its CPU
    evaluator runs a joint) on one (b, h) instance at the full S, verified
    against the closed-form gradients from the same evaluation, reported in
    TFLOP/s of the GPU row's algorithmic count (2.5 x the causal forward)
    and extrapolated to the full config as 64 instances x that time. One lap
    (~10-20 s on 16 host cores)."""
    from oracle import region_eval as rev
    from pdum_dsl_amd.tl import zoo
    from pdum_dsl_amd.tl.autodiff import grad, region_names

    B, H, S, D = 4, 16, 2048, 64
    subj = zoo.attention(T=S, S=S, E=D, OD=D, mask="causal", seed=5, scale=D**-0.5)
    rg = grad(subj.region, "out", seed="dO", names=region_names(subj.region, ("q", "k", "v"), ("out",)))
    dO = np.random.default_rng(6).standard_normal((S, D))
    vals = [rev.value(a, p.type) for a, p in zip(subj.numpy_inputs() + [dO], rg.region.params)]
    t0 = time.perf_counter()
    res = rev.evaluate(rg.region, vals)
    sec = time.perf_counter() - t0
    q, k, v = subj.numpy_inputs()
    wq, wk, wv = cf.attention_bwd(q, k, v, dO, scale=1.0, band=(None, 0))
    err = max(float(np.abs(res[1].numpy(("t", "e")) - wq).max()), float(np.abs(res[2].numpy(("s", "e")) - wk).max()),
              float(np.abs(res[3].numpy(("s", "o")) - wv).max()))
    assert err < 1e-9, f"C5 CPU row disagrees with the closed-form gradients: {err}"
    del res
    fl = 2.5 * causal_flops(1, 1, S, D)
    n_inst = B * H
    return {"config": "C5 causal bwd B=4 H=16 S=2048 D=64: one (b, h) instance, extrapolated",
            "template": "grad joint (naive twin)", "value": round(fl / sec / 1e12, 8), "unit": "TFLOP/s",
            "ms_one_instance": round(sec * 1e3, 1), "laps": 1, "max_abs_err": err,
            "extrapolated_full_ms": round(sec * n_inst * 1e3, 1),
            "extrapolation": f"{n_inst} (b, h) instances x the one-instance time", **host}


def cpu_baseline(cf):
    """The reference's CPU path restated — the flash template's generated tile
    program (fusion.plan_region over the naive attention region, the online-
    softmax fold of fusion.py:542-615) evaluated by the float64 region
    interpreter (oracle.region_eval: dense per-node evaluation, the fold as a
    Python loop, as dialect.run_region / the torch-CPU Evaluator run it) — on
    a bounded sample of C3: one (b, h) instance, its first R query rows against
    their causal keys, repeated for ~10 s on this host's cores; reported as
    TFLOP/s of the same causal algorithmic count the GPU line uses. ``rows``
    adds C1 and C2 whole, the same way."""
    from oracle import region_eval as rev
    from pdum_dsl_amd.tl import zoo

    host = host_facts()
    R, D = 1024, 128
    subj = zoo.attention(T=R, S=R, E=D, OD=D, mask="causal", seed=3, scale=D**-0.5)
    g = _tile_program(subj.region)
    vals = [rev.value(f.arr, p.type) for f, p in zip(subj.inputs, g.kernel.params)]
    want = cf.attention(*subj.numpy_inputs(), scale=1.0, band=(None, 0))[0]
    t0 = time.perf_counter()
    reps = 0
    while True:
        out = rev.evaluate(g.kernel, vals)
        reps += 1
        if time.perf_counter() - t0 > 10.0:
            break
    el = time.perf_counter() - t0
    err = float(np.abs(out.numpy(("t", "o")) - want).max())
    assert err < 1e-9, f"CPU baseline disagrees with the closed form: {err}"  # verify-before-report
    fl = 4.0 * D * (R * (R + 1) / 2) * reps
    rate = fl / el
    full = causal_flops(8, 32, 4096, D)
    return {
        "value": round(rate / 1e12, 8),
        "unit": "TFLOP/s",
        "cores": host["torch_threads"],
        "kind": "port",
        "sample": f"oracle.region_eval (float64 torch-CPU interpreter) of the generated flash tile program "
        f"(si={dict(g.params)['si']}) on one C3 head, query rows [0,{R}) x their causal keys, {reps} reps in "
        f"{el:.1f} s",
        "extrapolated_full_ms": round(full / rate * 1e3, 1),
        "extrapolation": "the full C3 config's algorithmic FLOP (8 x 32 heads, 4096 causal rows) at the sample's "
        "rate",
        **host,
        "rows": cpu_rows(cf, host),
    }


def gemm_reference(torch, dev):
    """A plain bf16 GEMM through torch (hipBLASLt) on the same device: the
    practical MFMA ceiling the attention kernels are read against."""
    n = 16384
    a = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    b = torch.randn(n, n, device=dev, dtype=torch.bfloat16)
    ms = time_events(lambda: a @ b, 5, warmup=2)
    return {"op": f"torch.matmul bf16 {n}x{n}x{n}", "ms": round(ms, 4), "TFLOP/s": round(2 * n**3 / ms / 1e9, 1)}


if __name__ == "__main__":
    main()
