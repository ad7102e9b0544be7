"""Byte model of the ReplaySSM GDN decode path (HBM bytes per call).

Two accountings:

* ``algorithmic``: every compulsory tensor element counted once per call
  (checkpoint codes + scales, query, the ``fill`` ring tokens, output; a
  flush also writes the checkpoint back). This is the figure the roofline
  fraction is computed from:
      C = B*HV*V*K (fp8)       S = B*HV*(V/32)*2       Q = B*H*K*2
      O = B*HV*V*2             R = B*(H*K*2 + HV*V*2 + HV*2*2) per ring token
      replay(l) = C + S + Q + l*R + O
      flush(L)  = 2C + 2S + Q + L*R + O
      prep      = B*(2HK + HV*V)*2 + 2*B*HV*sizeof(a) + HV*8 + B*4 + Q + R
      full-contract per step = [sum_{l=1}^{L-1} replay(l) + flush(L) + L*prep] / L
* ``reference``: the reference's own per-call accounting, restated from
  prototype/bench_gdn_replayssm.py:45-87 (``traffic_bytes``: ring always
  full, no output term, query/keys re-read per V tile in ``replay_actual``),
  kept so ratios can be quoted on the reference's terms.

The bf16 read-modify-write comparison is B*HV*V*K*2*2 bytes per step
(state read + write, prototype/bench_gdn_replayssm.py:82).
"""

from __future__ import annotations

from dataclasses import dataclass

VBLOCK = 32


@dataclass(frozen=True)
class LayerShape:
    batch: int
    heads: int = 16          # H, key heads
    value_heads: int = 32    # HV
    key_dim: int = 128       # K
    value_dim: int = 128     # V
    act_bytes: int = 2       # q / ring / out storage (bf16)
    gate_bytes: int = 2      # a, b raw gating inputs (bf16)

    @property
    def checkpoint(self) -> int:
        return self.batch * self.value_heads * self.value_dim * self.key_dim

    @property
    def scales(self) -> int:
        return self.batch * self.value_heads * (self.value_dim // VBLOCK) * 2

    @property
    def query(self) -> int:
        return self.batch * self.heads * self.key_dim * self.act_bytes

    @property
    def output(self) -> int:
        return self.batch * self.value_heads * self.value_dim * self.act_bytes

    @property
    def ring_token(self) -> int:
        """k + v + g + beta of one token for the whole batch."""
        return self.batch * (self.heads * self.key_dim * self.act_bytes
                             + self.value_heads * self.value_dim * self.act_bytes
                             + self.value_heads * 2 * self.act_bytes)

    @property
    def mixed_row(self) -> int:
        return (2 * self.heads * self.key_dim + self.value_heads * self.value_dim) * self.act_bytes


def replay_bytes(s: LayerShape, fill: int, flush: bool) -> int:
    """Algorithmic bytes of one gdn_replay_fp8 call with ring fill ``fill``."""
    base = s.query + fill * s.ring_token + s.output
    if flush:
        return 2 * s.checkpoint + 2 * s.scales + base
    return s.checkpoint + s.scales + base


def prep_bytes(s: LayerShape) -> int:
    """Algorithmic bytes of one gdn_prep_ring call: mixed_qkv row, a, b,
    A_log + dt_bias (f32), pos (i32) read; q_out and one ring slot written."""
    return (s.batch * s.mixed_row + 2 * s.batch * s.value_heads * s.gate_bytes + s.value_heads * 8
            + s.batch * 4 + s.query + s.ring_token)


def cycle_bytes_per_step(s: LayerShape, window: int, with_prep: bool = True) -> float:
    """Full-contract (with_prep) or core bytes per decode step, averaged over
    one ring cycle: fills 1..window-1 replay, fill == window flushes."""
    total = sum(replay_bytes(s, fill, False) for fill in range(1, window)) + replay_bytes(s, window, True)
    if with_prep:
        total += window * prep_bytes(s)
    return total / window


def bf16_rmw_bytes(s: LayerShape) -> int:
    """State bytes of a bf16 read-modify-write decode step."""
    return s.batch * s.value_heads * s.value_dim * s.key_dim * 2 * 2


def reference_traffic(s: LayerShape, window: int, block_v: int) -> dict:
    """The reference's accounting (prototype/bench_gdn_replayssm.py:45-87)."""
    tiles = s.value_dim // block_v
    checkpoint = s.checkpoint
    scales = s.batch * s.value_heads * tiles * 2
    query = s.query
    ring_key = s.batch * window * s.heads * s.key_dim * 2
    ring_value = s.batch * window * s.value_heads * s.value_dim * 2
    ring_scalars = s.batch * window * s.value_heads * 4
    out = {
        "replay_logical": checkpoint + scales + query + ring_key + ring_value + ring_scalars,
        "replay_actual": checkpoint + scales + tiles * (query + ring_key) + ring_value + ring_scalars,
        "flush_actual": 2 * checkpoint + 2 * scales + tiles * ring_key + ring_value + ring_scalars,
        "bf16_baseline": bf16_rmw_bytes(s),
    }
    # one ring cycle: L - 1 replays and one flush (bench_gdn_replayssm.py:348-353)
    out["amortized_actual"] = (out["replay_actual"] * (window - 1) + out["flush_actual"]) / window
    out["amortized_logical"] = (out["replay_logical"] * (window - 1) + out["flush_actual"]) / window
    return out


# ---------------------------------------------------------------------------
# Measured traffic: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE reduction
# ---------------------------------------------------------------------------

def _counter_rows(run_dir):
    """(dispatch_id, kernel_name, counter_name, value) of every
    *counter_collection.csv under ``run_dir`` (rocprofv3 --output-format csv)."""
    import csv
    from pathlib import Path

    files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no *counter_collection.csv under {run_dir}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], r["Counter_Name"], float(r["Counter_Value"])))
    return rows


def _per_dispatch(rows, counter):
    """Counter value per dispatch (summed over the dimensions rocprofv3 reports)."""
    out = {}
    names = {}
    for dispatch, name, cname, value in rows:
        if cname != counter:
            continue
        out[dispatch] = out.get(dispatch, 0.0) + value
        names[dispatch] = name
    return out, names


def reduce_pmc(fetch_dir, write_dir, kernel: str, calib_bytes: int, calib_copies: int) -> dict:
    """HBM bytes per launch of ``kernel`` from two rocprofv3 --pmc runs of the
    same command (FETCH_SIZE, then WRITE_SIZE; KiB per dispatch). The command
    ends with ``calib_copies`` plain device copies of ``calib_bytes`` bytes;
    those last dispatches calibrate each counter (bytes the copy must move /
    KiB the counter reports), and the kernel's mean KiB per dispatch is scaled
    by that factor."""
    result = {"kernel": kernel, "calibration": {"copy_bytes": calib_bytes, "copies": calib_copies}}
    total = 0.0
    for label, run_dir, counter in (("fetch", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")):
        values, names = _per_dispatch(_counter_rows(run_dir), counter)
        order = sorted(values)
        calib = order[-calib_copies:]
        calib_kib = sum(values[d] for d in calib) / len(calib)
        factor = calib_bytes / (calib_kib * 1024.0)
        launches = [d for d in order if kernel in names[d]]
        if not launches:
            raise ValueError(f"no dispatch of {kernel!r} in {run_dir}")
        kib = sum(values[d] for d in launches) / len(launches)
        by_bytes = kib * 1024.0 * factor
        total += by_bytes
        result[label] = {
            "counter": counter,
            "kernel_dispatches": len(launches),
            "kernel_kib_per_dispatch": kib,
            "copy_kernel": names[calib[0]],
            "copy_kib_per_dispatch": calib_kib,
            "factor": factor,
            "bytes_per_launch": by_bytes,
        }
    result["bytes_per_launch"] = total
    return result


RDREQ_COUNTERS = ("TCC_EA0_RDREQ_sum", "TCC_EA0_RDREQ_32B_sum", "TCC_EA0_RDREQ_64B_sum", "TCC_EA0_RDREQ_128B_sum")


def reduce_rdreq(run_dir, kernel: str, calib_bytes: int, calib_copies: int) -> dict:
    """Read bytes per launch of ``kernel`` from the L2-to-memory read request
    counts of one rocprofv3 --pmc run (RDREQ_COUNTERS): 32 n_32B + 64 n_64B +
    128 n_128B bytes per dispatch, with no calibration factor. The last
    ``calib_copies`` dispatches are plain copies of ``calib_bytes``; their
    figure shows whether the three sizes account for every request and byte
    (a cross-check of the FETCH_SIZE calibration)."""
    rows = _counter_rows(run_dir)
    per = {}
    names = {}
    for dispatch, name, cname, value in rows:
        if cname in RDREQ_COUNTERS:
            per.setdefault(dispatch, {})[cname] = per.get(dispatch, {}).get(cname, 0.0) + value
            names[dispatch] = name
    order = sorted(per)

    def stats(ds):
        tot = {c: sum(per[d].get(c, 0.0) for d in ds) / len(ds) for c in RDREQ_COUNTERS}
        n_all, n32, n64, n128 = (tot[c] for c in RDREQ_COUNTERS)
        return {"requests": n_all, "req_32B": n32, "req_64B": n64, "req_128B": n128,
                "unsized_requests": n_all - n32 - n64 - n128, "bytes": 32 * n32 + 64 * n64 + 128 * n128}

    calib = stats(order[-calib_copies:])
    launches = [d for d in order if kernel in names[d]]
    if not launches:
        raise ValueError(f"no dispatch of {kernel!r} in {run_dir}")
    res = stats(launches)
    return {"kernel": kernel, "dispatches": len(launches), **res,
            "copy": {**calib, "expected_bytes": calib_bytes, "bytes_over_expected": calib["bytes"] / calib_bytes}}


def trace_by_fill(run_dir, kernel: str, sets: int, window: int, rounds: int = 2) -> dict:
    """Launch durations of ``kernel`` by ring fill from a rocprofv3
    --kernel-trace run of ``bench.py --profile``: the last ``rounds`` rounds
    of sets x window launches, launch i at fill (i // sets) % window + 1 (the
    bench's cycle). Returns {fill: (mean, min, max) us}, the cycle mean, and
    the median gap between consecutive launches."""
    import csv
    import statistics
    from pathlib import Path

    files = sorted(Path(run_dir).rglob("*kernel_trace.csv"))
    if not files:
        raise FileNotFoundError(f"no *kernel_trace.csv under {run_dir}")
    rows = []
    for f in files:
        with open(f, newline="") as fh:
            rows += [r for r in csv.DictReader(fh) if kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    last = rows[-rounds * sets * window:]
    if len(last) < rounds * sets * window:
        raise ValueError(f"{len(rows)} launches of {kernel!r}, fewer than {rounds} rounds")
    by = {f: [] for f in range(1, window + 1)}
    for i, r in enumerate(last):
        by[(i // sets) % window + 1].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    table = {f: (statistics.mean(v), min(v), max(v)) for f, v in by.items()}
    gaps = [(int(b["Start_Timestamp"]) - int(a["End_Timestamp"])) / 1e3 for a, b in zip(last, last[1:])]
    return {"by_fill": table, "cycle_mean_us": statistics.mean(m for m, _, _ in table.values()),
            "gap_median_us": statistics.median(gaps), "kernel": rows[-1]["Kernel_Name"]}


if __name__ == "__main__":
    import argparse
    import json
    import sys

    if "--rdreq" in sys.argv:
        p = argparse.ArgumentParser(description="Read bytes per launch from L2-to-memory request counts")
        p.add_argument("--rdreq", required=True, help="rocprofv3 -d directory of the RDREQ_COUNTERS run")
        p.add_argument("--kernel", default="decode_kernel", help="substring of the kernel name")
        p.add_argument("--calib-bytes", type=int, default=64 << 20)
        p.add_argument("--calib-copies", type=int, default=4)
        p.add_argument("--out", default=None)
        args = p.parse_args()
        res = reduce_rdreq(args.rdreq, args.kernel, args.calib_bytes, args.calib_copies)
        if args.out:
            with open(args.out, "w") as fh:
                json.dump(res, fh, indent=1)
                fh.write("\n")
        print(json.dumps(res, indent=1))
        sys.exit(0)
    if "--trace" in sys.argv:
        p = argparse.ArgumentParser(description="Launch durations by ring fill from a rocprofv3 kernel trace")
        p.add_argument("--trace", required=True, help="rocprofv3 -d directory of the --kernel-trace run")
        p.add_argument("--kernel", default="decode_kernel", help="substring of the kernel name")
        p.add_argument("--sets", type=int, default=12)
        p.add_argument("--window", type=int, default=16)
        args = p.parse_args()
        res = trace_by_fill(args.trace, args.kernel, args.sets, args.window)
        print(f"kernel: {res['kernel']}")
        print("| fill | " + " | ".join(str(f) for f in res["by_fill"]) + " |")
        print("|---" * (len(res["by_fill"]) + 1) + "|")
        for k, name in enumerate(("mean us", "min us", "max us")):
            print(f"| {name} | " + " | ".join(f"{v[k]:.2f}" for v in res["by_fill"].values()) + " |")
        print(f"cycle mean {res['cycle_mean_us']:.2f} us per launch; median gap between launches "
              f"{res['gap_median_us']:.2f} us")
        sys.exit(0)

    p = argparse.ArgumentParser(description="Reduce rocprofv3 FETCH_SIZE / WRITE_SIZE runs to HBM bytes per launch")
    p.add_argument("--fetch", required=True, help="rocprofv3 -d directory of the FETCH_SIZE run")
    p.add_argument("--write", required=True, help="rocprofv3 -d directory of the WRITE_SIZE run")
    p.add_argument("--kernel", default="decode_kernel", help="substring of the kernel name")
    p.add_argument("--calib-bytes", type=int, default=64 << 20)
    p.add_argument("--calib-copies", type=int, default=4)
    p.add_argument("--algorithmic-bytes", type=float, default=None,
                   help="algorithmic bytes per launch, recorded beside the measured figure")
    p.add_argument("--out", required=True)
    args = p.parse_args()
    res = reduce_pmc(args.fetch, args.write, args.kernel, args.calib_bytes, args.calib_copies)
    if args.algorithmic_bytes:
        res["algorithmic_bytes_per_launch"] = args.algorithmic_bytes
        res["traffic_over_algorithmic"] = res["bytes_per_launch"] / args.algorithmic_bytes
    with open(args.out, "w") as fh:
        json.dump(res, fh, indent=1)
        fh.write("\n")
    print(json.dumps(res, indent=1))
