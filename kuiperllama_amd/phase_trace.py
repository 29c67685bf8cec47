"""Per-phase device-time breakdown of the persistent decode step.

    python -m kuiperllama_amd.phase_trace <config> [positions] [repeats]

runs kl_engine_trace_step (one persistent launch with per-workgroup
s_memrealtime marks: kernel entry, then per phase "input staged" and
"outputs stored") on a synthetic image of a BASELINE/TINY config at each
position (comma-separated, default 200) and prints, per phase kind, the
averages over the model's layers and the repeats, in microseconds:

  cp       critical path: last workgroup done in this phase - last done in
           the previous one (kernel entry for the first phase);
  handoff  last workgroup's input staged - last done in the previous phase;
  work     staged -> done per workgroup: median and maximum;
  tail     last done - median done.

The sum of the critical paths is the step's device time.  Positions are
traced on a fresh cache (the timing does not depend on the cache contents).
"""
from __future__ import annotations

import sys

import numpy as np

from . import ALL, Engine, synth_image

PHASES = ["qkv", "attn", "wo", "w13", "w2"]
TICK_US = 0.01  # s_memrealtime: 100 MHz


def breakdown(eng: Engine, layers: int, pos: int, repeats: int = 3) -> dict:
    """{phase kind: [cp, handoff, work median, work max, tail]} averaged
    over layers and repeats, plus "step" (mean device time of the step)."""
    nph = 5 * layers + 1
    acc: dict[str, np.ndarray] = {}
    steps = []
    for _ in range(repeats):
        tr = eng.trace_step(5, pos).astype(np.float64) * TICK_US
        entry = tr[0]
        done_prev = entry.max()
        steps.append(tr[2 * nph].max() - entry.min())
        for p in range(nph):
            st, dn = tr[2 * p + 1], tr[2 * p + 2]
            kind = "cls" if p == nph - 1 else PHASES[p % 5]
            row = np.array([dn.max() - done_prev, st.max() - done_prev, np.median(dn - st),
                            (dn - st).max(), dn.max() - np.median(dn), 1.0])
            acc[kind] = acc.get(kind, np.zeros(6)) + row
            done_prev = dn.max()
    out = {k: (v[:5] / v[5]).tolist() + [v[0] / repeats] for k, v in acc.items()}
    out["step"] = float(np.mean(steps))
    return out


def main(argv: list[str]) -> int:
    if not argv or argv[0] not in ALL:
        print(__doc__)
        print("configs:", ", ".join(ALL))
        return 2
    cfg = ALL[argv[0]]
    positions = [int(x) for x in (argv[1] if len(argv) > 1 else "200").split(",")]
    repeats = int(argv[2]) if len(argv) > 2 else 3
    eng = Engine(synth_image(cfg), cfg)
    print(f"# {cfg.name}: {cfg.layers} layers, launch {eng.launch_shape()}", flush=True)
    for pos in positions:
        b = breakdown(eng, cfg.layers, pos, repeats)
        print(f"position {pos}: step {b.pop('step'):.1f} us")
        print("  phase   cp/phase  handoff  work med  work max   tail   cp total")
        total = 0.0
        for kind, (cp, ho, wm, wx, tail, cp_tot) in b.items():
            print(f"  {kind:5s} {cp:9.2f} {ho:8.2f} {wm:9.2f} {wx:9.2f} {tail:6.2f} {cp_tot:9.1f}")
            total += cp_tot
        print(f"  sum of critical paths {total:.1f} us", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
