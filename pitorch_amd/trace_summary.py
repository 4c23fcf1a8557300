"""Per-phase summary of a Chrome-Tracing JSON trace in the reference's
format (pt_trace_write_json; pitorch/profiler/trace.c:67-98): for each span
(category, name; layer spans L<l>_<name> pooled over layers) the number of
spans per step, the mean duration and the time per step, with the share
of the mean train_step.

    python -m pitorch_amd.trace_summary trace.json
"""
import collections
import json
import re
import sys


def summarize(events):
    steps = [e for e in events if e["name"] == "train_step"]
    n_steps = max(1, len(steps))
    step_us = sum(e["dur"] for e in steps) / n_steps if steps else 0.0
    acc = collections.OrderedDict()
    for e in events:
        m = re.match(r"L(\d+)_(.*)$", e["name"])
        key = (e["cat"], m.group(2) if m else e["name"], bool(m))
        acc.setdefault(key, []).append(e["dur"])
    rows = []
    for (cat, name, per_layer), durs in acc.items():
        per_step = sum(durs) / n_steps
        rows.append((cat, ("L*_" if per_layer else "") + name, len(durs) / n_steps, sum(durs) / len(durs), per_step,
                     100.0 * per_step / step_us if step_us else 0.0))
    return n_steps, step_us, rows


def main(argv):
    if len(argv) != 2:
        print(__doc__.strip(), file=sys.stderr)
        return 2
    n_steps, step_us, rows = summarize(json.load(open(argv[1])))
    print(f"{n_steps} train_step spans, mean {step_us:.1f} us\n")
    print("| cat | span | per step | mean us | us per step | % of train_step |")
    print("|---|---|---:|---:|---:|---:|")
    for cat, name, cnt, mean, per_step, pct in rows:
        print(f"| {cat} | {name} | {cnt:g} | {mean:.1f} | {per_step:.1f} | {pct:.1f} |")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
