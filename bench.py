"""Benchmark of the MoE FFN block on one MI355X.

Workload ("C2"): Mixtral-8x7B-shaped moe_ffn_block,
bf16 activations and weights, fp32 accumulation, hidden 4096, ffn 14336,
8 experts, top-2, no renormalisation.  A step is one moe_ffn_block call on
4096 tokens already resident in HBM (prefill); the 16-token decode call is
measured the same way and reported under "decode".  Inputs are synthetic and
seeded (frank-models_amd/workloads.py): activations N(0,1), weights
N(0,0.02^2), router rows redrawn until the top-3 probabilities are >= 1e-3
apart.

The JSON line carries:
  value / ms_per_step   whole-block throughput (tokens/s) over --steps calls,
                        bracketed by torch.cuda.synchronize()
  roofline              the dominant kernel (grouped gate+up GEMM), its
                        average duration from HIP events recorded by the
                        library on the launch stream, algorithmic FLOPs per
                        launch (useful work only) against the dense bf16 MFMA
                        peak (2.5 PFLOP/s); traffic from rocprofv3 PMC
                        counters when a summary is committed, else null
  block_mfma_frac       block FLOPs (2*T*H*E + 6*T*k*H*F) / step time / peak
  decode                T=16: tokens/s and block HBM fraction (bytes of the
                        touched experts' weights + activations / time / 8 TB/s)
  cpu_baseline          the oracle's expert-grouped NumPy restatement (oracle/)
                        timed on this host on a bounded token sample
  attention_decode      the decode step's attention half at Mixtral's attention
                        shape (16 sequences x 4096 cached positions, paged
                        bf16 KV): ms/step, per-phase times, KV-read GB/s;
                        decode_layer: that attention sub-layer followed by the
                        C2 MoE sub-layer on the same 16 tokens
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_BF16_FLOPS = 2.5e15
PEAK_HBM_BYTES = 8.0e12
METRIC = "MoE FFN tokens/s + % MFMA peak (prefill) / % HBM BW (decode), Mixtral-shape"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def block_flops(T, H, F, E, k):
    return 2.0 * T * H * E + 6.0 * T * k * H * F


def block_bytes(T, H, F, E, k, touched, wbytes=2, abytes=2):
    return touched * 3.0 * H * F * wbytes + E * H * abytes + 2.0 * T * H * abytes + 2.0 * T * k * 4


def run_config(fm, wl, torch, cfg, T, steps, warmup, weights=None, sublayer=False):
    """Times `steps` block calls at T tokens (and, with `sublayer`, the
    norm + block + residual sub-layer); returns a dict of measurements."""
    x_np, wr_np, gen = wl.router_inputs(cfg, T)
    x = torch.from_numpy(x_np).to("cuda", torch.bfloat16)
    wr = torch.from_numpy(wr_np).to("cuda", torch.bfloat16)
    if weights is None:
        t0 = time.perf_counter()
        dev_w = wl.expert_weights(cfg, "cuda", dtype=torch.bfloat16)
        torch.cuda.synchronize()
        log(f"weights drawn in {time.perf_counter() - t0:.1f}s")
        t0 = time.perf_counter()
        if cfg.weights == "fp8":
            packed = [fm.quantize_expert_weights(w) for w in dev_w]
        else:
            packed = [fm.pack_expert_weights(w) for w in dev_w]
        torch.cuda.synchronize()
        pack_s = time.perf_counter() - t0
        weights = (dev_w, packed, pack_s)
    dev_w, packed, pack_s = weights
    block = fm.MoEFFNBlock(wr, *packed, cfg.n_expert, cfg.n_expert_used, cfg.n_embd, cfg.n_ff,
                           cfg.normalize, act_dtype=torch.bfloat16)
    out = torch.empty((T, cfg.n_embd), dtype=torch.bfloat16, device="cuda")
    for _ in range(warmup):
        block(x, out=out)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        block(x, out=out)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # Per-kernel durations: HIP events recorded by the library on the launch stream.
    ll = fm.lowlevel
    ll.timing_read()
    ll.timing_enable(True)
    for _ in range(steps):
        block(x, out=out)
    torch.cuda.synchronize()
    kernels = ll.timing_read()
    ll.timing_enable(False)
    ids = block.routing(T)[0]
    touched = int(torch.unique(ids).numel())
    res = dict(T=T, elapsed=elapsed, ms=elapsed / steps * 1e3, tok_s=steps * T / elapsed,
               kernels={k: (v[0] / v[1] if v[1] else 0.0) for k, v in kernels.items() if v[1]},
               touched=touched, pack_s=pack_s, gen=gen, x_np=x_np, wr_np=wr_np, weights=weights)
    if sublayer:
        # The MoE FFN sub-layer on the same batch as residual stream: ffn_norm,
        # block, residual add (unit norm weight; routing is not checked here).
        nw = torch.ones(cfg.n_embd, dtype=torch.bfloat16, device="cuda")
        sub_out = torch.empty_like(out)
        for _ in range(warmup):
            block.sublayer(x, nw, 1e-5, out=sub_out)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            block.sublayer(x, nw, 1e-5, out=sub_out)
        torch.cuda.synchronize()
        res["sublayer_ms"] = (time.perf_counter() - t0) / steps * 1e3
        ll.timing_read()
        ll.timing_enable(True)
        for _ in range(steps):
            block.sublayer(x, nw, 1e-5, out=sub_out)
        torch.cuda.synchronize()
        k2 = ll.timing_read()
        ll.timing_enable(False)
        res["sublayer_kernels"] = {k: (v[0] / v[1] if v[1] else 0.0) for k, v in k2.items() if v[1]}
    return res


def cpu_baseline(torch, cfg, res, sample):
    """Expert-grouped NumPy restatement (oracle/) on `sample` tokens of the
    same batch, fp32, on this host's cores."""
    import numpy as np
    from oracle import moe as om

    dev_w = res["weights"][0]
    host_w = [w.float().cpu().numpy() for w in dev_w]
    xs = res["x_np"][:sample]
    try:
        from threadpoolctl import threadpool_info

        threads = max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:  # pragma: no cover - reporting only
        threads = len(os.sched_getaffinity(0))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        om.moe_ffn_block(xs, res["wr_np"], *host_w, cfg.n_expert, cfg.n_expert_used, cfg.n_embd, cfg.n_ff,
                         cfg.normalize, dtype=np.float32)
        times.append(time.perf_counter() - t0)
    best = min(times)
    return {
        "value": sample / best,
        "unit": "tokens/s",
        "cores": int(threads),
        "kind": "port",
        "sample": (f"{sample} of the {res['T']} tokens, fp32 expert-grouped NumPy/OpenBLAS restatement of "
                   f"oracles/moe.py (oracle/moe.py), best of {len(times)} runs ({best:.2f}s each)"),
    }


def all_configs(fm, wl, torch, args):
    """Every BASELINE configuration and token count: ms/step, tokens/s, block
    MFMA fraction (bf16/fp8 peak) and HBM fraction of the touched weights."""
    rows = []
    for name in ("C2", "C3", "C4", "C5"):
        cfg = wl.CONFIGS[name]
        H, F, E, k = cfg.n_embd, cfg.n_ff, cfg.n_expert, cfg.n_expert_used
        weights = None
        for T in cfg.tokens:
            res = run_config(fm, wl, torch, cfg, T, max(5, args.steps // 2), 5, weights=weights, sublayer=True)
            weights = res["weights"]
            wb = 1 if cfg.weights == "fp8" else 2
            flops = block_flops(T, H, F, E, k)
            nbytes = block_bytes(T, H, F, E, k, res["touched"], wbytes=wb)
            row = {"config": name, "tokens": T, "ms": res["ms"], "tokens_per_s": res["tok_s"],
                   "mfma_frac": flops / (res["ms"] * 1e-3) / PEAK_BF16_FLOPS,
                   "hbm_frac": nbytes / (res["ms"] * 1e-3) / PEAK_HBM_BYTES,
                   "experts_touched": res["touched"], "kernels_ms": res["kernels"],
                   "sublayer_ms": res["sublayer_ms"], "sublayer_kernels_ms": res["sublayer_kernels"]}
            rows.append(row)
            log(f"{name} T={T:5d}: {res['ms']:.3f} ms  {res['tok_s']:.0f} tok/s  mfma {row['mfma_frac']:.3f}  "
                f"hbm {row['hbm_frac']:.3f}  {res['kernels']}")
            log(f"{name} T={T:5d}: sub-layer {res['sublayer_ms']:.3f} ms  "
                f"norm {res['sublayer_kernels'].get('norm', 0.0):.4f} ms  "
                f"combine {res['sublayer_kernels'].get('combine', 0.0):.4f} ms")
        del weights
        torch.cuda.empty_cache()
    return rows


def attention_decode(fm, torch, batch, ctx, steps, warmup, block_size=16, cpu_sample=0, moe=None):
    """The decode step's attention half at Mixtral-8x7B's attention shape
    (n_embd 4096, 32 query heads, 8 KV heads, head_dim 128), bf16: one new
    token per sequence for `batch` sequences, each with `ctx` cached
    positions in a paged pool (block_size rows per block, blocks shuffled),
    through AttentionBlockDecode.paged (projections, RoPE, attention read
    in place, output projection, scatter of the new K/V)."""
    n_embd, H, Hkv = 4096, 32, 8
    D = n_embd // H
    nkv = Hkv * D
    g = torch.Generator(device="cuda").manual_seed(7)
    bf = torch.bfloat16
    rnd = lambda *s, scale=1.0: (torch.randn(*s, generator=g, device="cuda") * scale).to(bf)
    per_seq = (ctx + 1 + block_size - 1) // block_size
    n_blocks = batch * per_seq
    kp = rnd(n_blocks, block_size, Hkv, D)
    vp = rnd(n_blocks, block_size, Hkv, D)
    perm = torch.randperm(n_blocks, generator=g, device="cuda").to(torch.int32)
    tables = perm.view(1, batch, per_seq).contiguous()
    lens = torch.full((1, batch), ctx, dtype=torch.int32, device="cuda")
    bi = tables[0, :, ctx // block_size].contiguous()
    pi = torch.full((batch,), ctx % block_size, dtype=torch.int32, device="cuda")
    s = n_embd ** -0.5
    blk = fm.AttentionBlockDecode(rnd(n_embd, n_embd, scale=s), rnd(n_embd, nkv, scale=s), rnd(n_embd, nkv, scale=s),
                                  rnd(n_embd, n_embd, scale=s), n_head=H, n_head_kv=Hkv, n_embd=n_embd, act_dtype=bf)
    x = rnd(batch, n_embd)
    pos = torch.full((batch,), ctx, dtype=torch.int64, device="cuda")

    def step():
        blk.paged(x, pos, kp, vp, 0, tables, lens, ctx, bi, pi)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    ll = fm.lowlevel
    ll.timing_read()
    ll.timing_enable(True)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    kern = {k: v[0] / v[1] for k, v in ll.timing_read().items() if v[1]}
    ll.timing_enable(False)
    kv_bytes = 2.0 * batch * ctx * nkv * 2
    qkv_bytes = n_embd * (n_embd + 2 * nkv) * 2.0
    out_bytes = n_embd * n_embd * 2.0
    res = {"workload": "Mixtral-8x7B attention (4096, 32 heads, 8 KV heads, head_dim 128), bf16, paged block 16",
           "batch": batch, "context": ctx, "ms_per_step": ms, "tokens_per_s": batch / (ms * 1e-3),
           "kernels_ms": kern, "kv_bytes": kv_bytes, "qkv_weight_bytes": qkv_bytes, "out_weight_bytes": out_bytes,
           "step_hbm_frac": (kv_bytes + qkv_bytes + out_bytes) / (ms * 1e-3) / PEAK_HBM_BYTES}
    if kern.get("attention"):
        res["attention_GBps"] = kv_bytes / (kern["attention"] * 1e-3) / 1e9
        res["attention_hbm_frac"] = res["attention_GBps"] * 1e9 / PEAK_HBM_BYTES
    if kern.get("qkv"):
        res["qkv_GBps"] = qkv_bytes / (kern["qkv"] * 1e-3) / 1e9
    if kern.get("out_proj"):
        res["out_proj_GBps"] = out_bytes / (kern["out_proj"] * 1e-3) / 1e9
    if moe is not None:
        # One whole decode layer body (transformer_layer_moe_decode.mlir:174-255):
        # the attention sub-layer then the MoE sub-layer, both in place on the
        # residual stream of the same `batch` tokens.
        wr, packed, cfg = moe
        moe_blk = fm.MoEFFNBlock(wr, *packed, cfg.n_expert, cfg.n_expert_used, cfg.n_embd, cfg.n_ff,
                                 cfg.normalize, act_dtype=bf)
        resid = rnd(batch, n_embd)
        nw = torch.ones(n_embd, dtype=bf, device="cuda")

        def layer():
            blk.paged_sublayer(resid, nw, 1e-5, pos, kp, vp, 0, tables, lens, ctx, bi, pi, out=resid)
            moe_blk.sublayer(resid, nw, 1e-5, out=resid)

        for _ in range(warmup):
            layer()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            layer()
        torch.cuda.synchronize()
        lms = (time.perf_counter() - t0) / steps * 1e3
        res["decode_layer"] = {"ms_per_step": lms, "tokens_per_s": batch / (lms * 1e-3),
                               "what": f"attention sub-layer ({batch} sequences x {ctx} positions) + MoE "
                                       f"sub-layer ({cfg.name}, {batch} tokens), in place on one residual stream"}
    if cpu_sample:
        res["cpu_baseline"] = attention_cpu_baseline(torch, blk, x, pos, kp, vp, tables, lens, ctx, bi, pi, cpu_sample)
    return res


def attention_cpu_baseline(torch, blk, x, pos, kp, vp, tables, lens, ctx, bi, pi, sample):
    """The oracle's gather + attention_block_decode + scatter (oracle/attention.py,
    NumPy float32) on `sample` of the sequences, timed on this host."""
    import numpy as np
    from oracle import attention as oa

    tb = tables[:, :sample].cpu().numpy()
    needed = np.unique(tb)
    remap = {int(b): i for i, b in enumerate(needed)}
    tb = np.vectorize(remap.get)(tb).astype(np.int32)
    kh = kp[torch.from_numpy(needed).cuda().long()].float().cpu().numpy()
    vh = vp[torch.from_numpy(needed).cuda().long()].float().cpu().numpy()
    ws = [torch.randn(s, device="cuda").mul(s[0] ** -0.5).float().cpu().numpy()
          for s in ((4096, 4096), (4096, 1024), (4096, 1024), (4096, 4096))]
    xs = x[:sample].float().cpu().numpy()
    ps = pos[:sample].cpu().numpy()
    bis = np.array([remap[int(b)] for b in bi[:sample].cpu().numpy()], np.int32)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oa.attention_decode_paged(xs, ps, kh, vh, 0, tb, lens[:, :sample].cpu().numpy(), ctx, bis,
                                  pi[:sample].cpu().numpy(), *ws, None, None, None, None, False, 32, 8, 4096,
                                  dtype=np.float32)
        times.append(time.perf_counter() - t0)
    dt = min(times)
    return {"value": sample / dt, "unit": "tokens/s", "cores": len(os.sched_getaffinity(0)), "kind": "port",
            "sample": f"{sample} of the {x.shape[0]} sequences ({ctx} cached positions each), fp32 NumPy gather + "
                      f"attention_block_decode + scatter (oracle/attention.py), best of {len(times)} runs "
                      f"({dt:.2f}s each), random weights of the same shapes"}


def read_traffic(kernel_name):
    """HBM bytes per launch of `kernel_name` from a committed rocprofv3 PMC
    summary (profiles/pmc_<name>.json), or None."""
    p = ROOT / "profiles" / f"pmc_{kernel_name}.json"
    if not p.exists():
        return None
    try:
        return float(json.loads(p.read_text())["hbm_bytes_per_launch"])
    except Exception:
        return None


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--tokens", type=int, default=4096)
    ap.add_argument("--decode-tokens", type=int, default=16)
    ap.add_argument("--cpu-sample", type=int, default=4096)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--attn-batch", type=int, default=16)
    ap.add_argument("--attn-context", type=int, default=4096)
    ap.add_argument("--no-attention", action="store_true")
    ap.add_argument("--attention-only", action="store_true",
                    help="time only the decode attention half (its own JSON line)")
    ap.add_argument("--all-configs", action="store_true",
                    help="also time C3/C4/C5 at every token count (table on stderr, 'configs' in the JSON)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the MoE FFN path here is built and timed on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured configuration); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    fm = importlib.import_module("frank-models_amd")
    wl = importlib.import_module("frank-models_amd.workloads")
    if args.attention_only:
        att = attention_decode(fm, torch, args.attn_batch, args.attn_context, max(args.steps, 20), args.warmup,
                               cpu_sample=0 if args.no_cpu_baseline else args.attn_batch)
        log(f"attention decode {att['ms_per_step']:.3f} ms/step, kernels(ms) {att['kernels_ms']}")
        print(json.dumps({"metric": "decode attention tokens/s (paged KV, Mixtral attention shape)",
                          "value": att["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1, "dtype": "bf16",
                          "data": "synthetic", "higher_is_better": True, "attention_decode": att}), flush=True)
        return
    cfg = wl.CONFIGS["C2"]
    H, F, E, k = cfg.n_embd, cfg.n_ff, cfg.n_expert, cfg.n_expert_used

    log(f"prefill T={args.tokens}: {args.warmup} warmup + {args.steps} timed steps")
    pre = run_config(fm, wl, torch, cfg, args.tokens, args.steps, args.warmup)
    log(f"prefill {pre['ms']:.3f} ms/step, {pre['tok_s']:.0f} tok/s, kernels(ms) {pre['kernels']}")

    T = args.tokens
    n_assign = T * k
    gu_ms = pre["kernels"].get("gate_up", 0.0)
    gu_flops = 2.0 * n_assign * H * (2 * F)
    achieved = gu_flops / (gu_ms * 1e-3) / 1e12 if gu_ms else 0.0
    roofline = {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s",
                "frac": achieved * 1e12 / PEAK_BF16_FLOPS, "traffic": read_traffic("gate_up_prefill"),
                "kernel": "gemm_tiled256_kernel<SWIGLU> (gate+up grouped GEMM, SwiGLU epilogue)",
                "kernel_ms": gu_ms, "flops_per_launch": gu_flops}
    flops = block_flops(T, H, F, E, k)
    result = {
        "metric": METRIC,
        "value": pre["tok_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["ms"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations, N(0,0.02^2) random-init weights of the Mixtral-8x7B MoE layer)",
        "config": {"workload": "C2 Mixtral-8x7B moe_ffn_block prefill", "tokens": T, "n_embd": H, "n_ff": F,
                   "n_expert": E, "n_expert_used": k, "normalize_weights": cfg.normalize,
                   "weights": "bf16", "accumulate": "fp32"},
        "roofline": roofline,
        "block_mfma_frac": flops / (pre["ms"] * 1e-3) / PEAK_BF16_FLOPS,
        "block_tflops": flops / (pre["ms"] * 1e-3) / 1e12,
        "kernels_ms": pre["kernels"],
        "pack_s": pre["pack_s"],
    }

    if not args.no_decode:
        Td = args.decode_tokens
        log(f"decode T={Td}")
        dec = run_config(fm, wl, torch, cfg, Td, max(args.steps, 20), args.warmup, weights=pre["weights"])
        nbytes = block_bytes(Td, H, F, E, k, dec["touched"])
        result["decode"] = {
            "tokens": Td, "tokens_per_s": dec["tok_s"], "ms_per_step": dec["ms"],
            "experts_touched": dec["touched"], "algorithmic_bytes": nbytes,
            "hbm_frac": nbytes / (dec["ms"] * 1e-3) / PEAK_HBM_BYTES,
            "achieved_GBps": nbytes / (dec["ms"] * 1e-3) / 1e9,
            "kernels_ms": dec["kernels"],
        }
        log(f"decode {dec['ms']:.3f} ms/step, {result['decode']['hbm_frac']:.3f} of HBM peak")

    if not args.no_attention:
        log(f"attention decode: batch {args.attn_batch}, context {args.attn_context}")
        wr = torch.from_numpy(pre["wr_np"]).to("cuda", torch.bfloat16)
        result["attention_decode"] = attention_decode(fm, torch, args.attn_batch, args.attn_context,
                                                      max(args.steps, 20), args.warmup,
                                                      cpu_sample=0 if args.no_cpu_baseline else args.attn_batch,
                                                      moe=(wr, pre["weights"][1], cfg))
        log(f"attention decode {result['attention_decode']['ms_per_step']:.3f} ms/step, "
            f"kernels(ms) {result['attention_decode']['kernels_ms']}")

    if args.all_configs:
        result["configs"] = all_configs(fm, wl, torch, args)

    if not args.no_cpu_baseline:
        log(f"cpu baseline on {args.cpu_sample} tokens")
        result["cpu_baseline"] = cpu_baseline(torch, cfg, pre, min(args.cpu_sample, T))
        log(f"cpu baseline {result['cpu_baseline']['value']:.1f} tok/s")
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
