"""Stage timeline of the persistent token kernel.

    python -m xpose_amd.trace [--ctx 4096] [--layers 26] [--seed S] [--repeat N]

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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--layers", type=int, default=26)
    ap.add_argument("--seed", type=lambda s: int(s, 0), default=0x5EED0003)
    ap.add_argument("--repeat", type=int, default=1)
    args = ap.parse_args()
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
