"""Stage timeline of the persistent token kernel, or (--batch) of the
persistent batched step kernel.

    python -m xpose_amd.trace [--ctx 4096] [--layers 26] [--seed S] [--repeat N]
    python -m xpose_amd.trace --batch [--repeat N]

Builds the seeded synthetic Gemma-3-1B model, pre-fills the KV cache to
position ctx (fp16 N(0,1)), decodes a few warm-up tokens, then records one
token with xp_session_trace and prints, per layer, how long each of the six
stages added to the critical path: the time from the previous stage's last
finisher to this stage's last finisher (100 MHz s_memrealtime stamps). That
increment is split into `wait` (previous stage's last finisher to the last
workgroup's input arrival: the exchange latency plus producer skew) and
`body` (last arrival to last finisher); `wg body` is the mean over working
workgroups of their own arrival-to-finish time. --repeat N records N
consecutive tokens and reports the means (and the spread of the total).
"""
from __future__ import annotations

import argparse

import numpy as np

STAGES = ("QKV", "attention", "combine", "O", "gate/up", "down")


def timeline(tr: np.ndarray, n_layers: int):
    """Per-layer stage increments (us), lm_head and argmax increments, total."""
    tr = tr.astype(np.int64)
    t0 = tr[0][tr[0] > 0].min()
    prev = 0.0
    rows = []
    for l in range(n_layers):
        inc = []
        for k in range(6):
            end = (tr[1 + 6 * l + k].max() - t0) / 100.0
            inc.append(end - prev)
            prev = end
        rows.append(inc)
    lm = (tr[6 * n_layers + 1].max() - t0) / 100.0
    am = (tr[6 * n_layers + 2].max() - t0) / 100.0
    return np.array(rows), lm - prev, am - lm, am


def arrivals(tr: np.ndarray, n_layers: int):
    """[n_layers][6][3]: wait, body and mean per-workgroup body (us) per stage."""
    tr = tr.astype(np.int64)
    t0 = tr[0][tr[0] > 0].min()
    out = np.zeros((n_layers, 6, 3))
    prev = 0.0
    for l in range(n_layers):
        for k in range(6):
            end = tr[1 + 6 * l + k]
            arr = tr[6 * n_layers + 3 + 6 * l + k]
            work = arr > 0
            end_max = (end.max() - t0) / 100.0
            if work.any():
                in_max = (arr[work].max() - t0) / 100.0
                wg_body = ((end[work] - arr[work]) / 100.0).mean()
            else:
                in_max, wg_body = end_max, 0.0
            out[l, k] = (in_max - prev, end_max - in_max, wg_body)
            prev = end_max
    return out


BATCH_STAGES = ("q|k|v", "attention", "o", "staging", "gate|up", "down", "staging")


def batch_main(repeat: int) -> int:
    """bench.py's config-5 workload (16 sequences at Philox depths in [128,
    4096], seeded synthetic Gemma-3-1B) through the persistent step kernel
    (XP_EXEC_TOKEN) with xp_batch_step_trace on: per stage, the mean wait
    (the stage before's last tile end to this stage's last input arrival)
    and body (that arrival to this stage's last tile end), local and global
    layers apart."""
    import xpose_amd as X
    X.init(0)
    cfg = X.XpConfig.gemma3_1b(max_seq=8192, sample_mode=1, temperature=0.8, top_k=64, top_p=0.95,
                               seed=0x5EED0005)
    sess = X.DecodeSession(cfg)
    sess.synthesize(0x5EED)
    n_seq, seed = 16, 0x5EED0005
    u = np.array([X.philox_uniform(seed, i, 0) for i in range(n_seq)])
    depths = (128 + np.floor(u * (4096 - 128 + 1))).astype(np.int64)
    b = X.DecodeBatch(sess, n_seq, 4096 + 40, X.XP_EXEC_TOKEN)
    kvd = cfg.n_kv_heads * cfg.head_dim
    dmax = int(depths.max())
    for l in range(cfg.n_layers):
        for which in (0, 1):
            rows = X.synth_normal_f16(dmax * kvd, seed, 2 * l + which)
            for i, d in enumerate(depths):
                b.kv_upload(i, l, which, 0, rows[:int(d) * kvd])
    b.set_positions(depths)
    b.forward(np.arange(n_seq) * 1000 + 7)
    for _ in range(3):
        b.decode_step()
    untraced = []
    for _ in range(5):
        b.decode_step()
        untraced.append(b.last_ms())
    b.step_trace(True)
    L, S = cfg.n_layers, len(BATCH_STAGES)
    acc = np.zeros((L, S, 2))
    kernel = []
    for _ in range(max(1, repeat)):
        b.decode_step()
        tr = b.step_trace_read().astype(np.int64)
        G = tr.size // (L * S * 2 + 1)
        t = tr[:L * S * 2 * G].reshape(L, S, 2, G)
        t0 = tr[L * S * 2 * G:].min()
        prev = t0
        for l in range(L):
            for k in range(S):
                has = t[l, k, 1] > 0
                ready, end = t[l, k, 0][has].max(), t[l, k, 1][has].max()
                acc[l, k] += ((ready - prev) / 100.0, (end - ready) / 100.0)
                prev = end
        kernel.append((prev - t0) / 100.0)
    b.step_trace(False)
    acc /= max(1, repeat)
    loc = [l for l in range(L) if not cfg.is_global(l)]
    glo = [l for l in range(L) if cfg.is_global(l)]
    print(f"step kernel: {np.mean(kernel):.1f} us traced; untraced step {np.mean(untraced):.4f} ms "
          f"(HIP events, {len(loc)} local + {len(glo)} global layers)")
    print(f"{'stage':10s} {'wait':>7s} {'body':>7s}   local (us)   {'wait':>7s} {'body':>7s}   global")
    for k, name in enumerate(BATCH_STAGES):
        lv, gv = acc[loc, k].mean(0), acc[glo, k].mean(0)
        print(f"{name:10s} {lv[0]:7.2f} {lv[1]:7.2f}   {'':10s}   {gv[0]:7.2f} {gv[1]:7.2f}")
    print(f"{'per layer':10s} {acc[loc].sum(axis=(1, 2)).mean():15.2f}   {'':10s}   "
          f"{acc[glo].sum(axis=(1, 2)).mean():15.2f}")
    b.close()
    sess.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=26)
    ap.add_argument("--seed", type=lambda s: int(s, 0), default=0x5EED0003)
    ap.add_argument("--repeat", type=int, default=1)
    ap.add_argument("--batch", action="store_true",
                    help="the persistent batched step kernel on the config-5 workload")
    args = ap.parse_args()
    if args.batch:
        return batch_main(args.repeat)
    import xpose_amd as X
    X.init(0)
    cfg = X.XpConfig.gemma3_1b(n_layers=args.layers, exec_mode=X.XP_EXEC_TOKEN)
    sess = X.DecodeSession(cfg)
    sess.synthesize(args.seed)
    kvd = cfg.n_kv_heads * cfg.head_dim
    for l in range(cfg.n_layers):
        sess.kv_upload(l, 0, 0, X.synth_normal_f16(args.ctx * kvd, args.ctx, 2 * l))
        sess.kv_upload(l, 1, 0, X.synth_normal_f16(args.ctx * kvd, args.ctx, 2 * l + 1))
    sess.set_position(args.ctx)
    sess.prefill([4242])
    sess.decode_steps(4)
    sess.trace(True)
    runs = []
    for _ in range(max(1, args.repeat)):
        sess.decode_steps(1)
        tr = sess.last_trace()
        runs.append((timeline(tr, cfg.n_layers), arrivals(tr, cfg.n_layers)))
    rows = np.mean([r[0][0] for r in runs], axis=0)
    lm = float(np.mean([r[0][1] for r in runs]))
    am = float(np.mean([r[0][2] for r in runs]))
    totals = np.array([r[0][3] for r in runs])
    total = float(totals.mean())
    glob = [l for l in range(cfg.n_layers) if cfg.is_global(l)]
    loc = [l for l in range(cfg.n_layers) if not cfg.is_global(l)]
    spread = f", min {totals.min():.1f} max {totals.max():.1f} over {len(runs)}" if len(runs) > 1 else ""
    print(f"token at position {args.ctx + 5}: {total:.1f} us{spread} "
          f"({len(loc)} local + {len(glob)} global layers)")
    print(f"{'stage':10s} {'local mean':>11s} {'global mean':>12s}   (us added to the critical path)")
    for k, name in enumerate(STAGES):
        lm_ = rows[loc, k].mean() if loc else float("nan")
        gm_ = rows[glob, k].mean() if glob else float("nan")
        print(f"{name:10s} {lm_:11.2f} {gm_:12.2f}")
    print(f"{'per layer':10s} {rows[loc].sum(1).mean() if loc else 0:11.2f} "
          f"{rows[glob].sum(1).mean() if glob else 0:12.2f}")
    arr = np.mean([r[1] for r in runs], axis=0)
    print(f"\n{'stage':10s} {'wait':>7s} {'body':>7s} {'wg body':>8s}   local layers (us)"
          f"   {'wait':>7s} {'body':>7s} {'wg body':>8s}   global layers")
    for k, name in enumerate(STAGES):
        lv = arr[loc, k].mean(0) if loc else np.full(3, np.nan)
        gv = arr[glob, k].mean(0) if glob else np.full(3, np.nan)
        print(f"{name:10s} {lv[0]:7.2f} {lv[1]:7.2f} {lv[2]:8.2f}   {'':13s}"
              f"   {gv[0]:7.2f} {gv[1]:7.2f} {gv[2]:8.2f}")
    print(f"lm_head    {lm:11.2f}\nargmax     {am:11.2f}")
    sess.close()
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
