"""Benchmark of the ReplaySSM GDN decode path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch 64] [--window 16]

Workload (BASELINE config 2 at its headline cell): the full-contract decode
step of one Qwen3.5-4B GDN layer (H=16, HV=32, K=V=128), batch 64, ring
window L=16, from raw bf16 mixed_qkv / a / b. A step is ONE launch of the
fused prep + replay kernel (gdn_prep_replay_fp8): q/k L2 norm, gating, ring
append, then the adjoint replay against the FP8 vblock32 checkpoint -- or, on
the ring's last slot, the forward rebuild + in-place requantisation (flush).
The batch runs the reference's cycle (prototype/bench_gdn_full_contract.py
:225-308): all sequences at ring fill l = 1..L, flushing at l = L, so the
per-step time is amortised over whole ring cycles.

Measurement:
  * BUFFER_SETS independent checkpoint + ring sets (~47 MB each at B=64) are
    used round-robin, one set per step, so consecutive steps never hit the
    256 MB Infinity Cache with the previous step's data; each set still runs
    a coherent cycle (set = step % S, fill = (step // S) % L + 1).
  * The steps are captured into a HIP graph (torch.cuda.CUDAGraph) once per
    round of S*L steps and replayed: no host launch overhead in the timed
    region. Timed = `steps` launches rounded up to whole rounds (so the cycle
    amortisation is exact), and never fewer than MIN_TIMED_ROUNDS rounds
    (>= 40 ms of launches at the headline, 3840 steps) whatever `--steps`
    asks: a short sample measures the clock ramp, not the kernel. The JSON
    reports the number of steps timed and the number requested.
  * Every timed section ends by reading the device word that counts bounded
    waits that gave up (gdnr_wait_timeouts); if any did, the step's results
    are meaningless and the benchmark prints an error instead of a figure.
  * HIP events on the launch stream bracket the timed region; `value` is
    microseconds per decode step (lower is better).
  * roofline: algorithmic bytes per step (every compulsory tensor element
    counted once; gdn_replayssm_traffic.cycle_bytes_per_step) / average launch
    duration, against 8 TB/s.
  * cpu_baseline: the reference's host algorithm (oracle/cpu_torch_path.py:
    dequantise -> forward replay -> emit, requantise on flush) in fp32 torch on
    the host cores, over one whole ring cycle of a batch sample, scaled to the
    full batch.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
PKG = REPO / "fp8-replayssm-gdn-kernel_amd"
for _p in (REPO, PKG):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "µs per GDN-layer decode step (B=64, L=16) + achieved HBM GB/s % of peak"
HBM_PEAK_GBS = 8000.0
# <tiles per row wave, row waves per head, ring chunks, fused, gate_f32, slots>
KERNEL_NAME = "decode_kernel<8, 1, 1, true, {gate_f32}, false>"
CPU_SAMPLE_SECONDS = 10.0
EXTRAS = ("core", "config1", "split", "config3", "floor")
CPU_MAX_CYCLES = 8
MIN_TIMED_ROUNDS = 20
MIN_WARM_ROUNDS = 2


class WaitTimeout(RuntimeError):
    """A decode workgroup's bounded LDS wait gave up during a timed section."""


def check_waits(section: str) -> None:
    """Raise WaitTimeout if any bounded wait gave up since the last check
    (gdnr_wait_timeouts; synchronises the device), and clear the word."""
    import gdnr_lib

    n = gdnr_lib.wait_timeouts(reset=True)
    if n:
        raise WaitTimeout(f"{section}: {n} bounded wait(s) gave up; the timed results are meaningless")


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3840)
    p.add_argument("--warmup", type=int, default=384)
    p.add_argument("--batch", type=int, default=64)
    p.add_argument("--window", type=int, default=16)
    p.add_argument("--block-v", type=int, default=128)
    p.add_argument("--sets", type=int, default=12, help="rotating buffer sets (defeats the Infinity Cache)")
    p.add_argument("--phase", choices=("lockstep", "mixed"), default="lockstep",
                   help="lockstep: the reference's cycle; mixed: sequence b at ring phase b %% L")
    p.add_argument("--cpu-sample", type=int, default=64, help="batch of the CPU-baseline sample (0: skip)")
    p.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    p.add_argument("--no-rmw", action="store_true",
                   help="skip the same-box timing of the bf16 read-modify-write comparator")
    p.add_argument("--trace", default=None,
                   help="capture file (the production hook's record format) to take the decode inputs from")
    p.add_argument("--trace-layer", type=int, default=0, help="layer of the capture file")
    p.add_argument("--no-mixed", action="store_true",
                   help="skip the same cycle timed again with staggered ring phases")
    p.add_argument("--no-slots", action="store_true",
                   help="skip the timing of the same cycle through the slot-indexed cache")
    p.add_argument("--profile", action="store_true",
                   help="short run for rocprofv3: no CPU baseline, few rounds")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the extra measurements (core-kernel cycles, config 1, split vs fused, config 3, "
                        "stream floor)")
    p.add_argument("--only", choices=EXTRAS, default=None,
                   help="run one extra measurement alone (no headline), e.g. under rocprofv3")
    return p.parse_args()


def traffic_from_profiles(batch: int, window: int):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel), as recorded in profiles/."""
    path = REPO / "profiles" / f"traffic_fused_b{batch}_l{window}.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def host_cpu() -> dict:
    """The host's CPU as lscpu reports it: model, sockets x cores x threads."""
    import subprocess

    info = {}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass

    def num(key):
        try:
            return int(info.get(key, ""))
        except ValueError:
            return None

    return {"model": info.get("Model name"), "sockets": num("Socket(s)"), "cores_per_socket": num("Core(s) per socket"),
            "threads_per_core": num("Thread(s) per core"), "logical_cpus": os.cpu_count()}


def cpu_baseline(args, shape, window):
    """Time the reference's host path on a batch sample; scale to the full batch."""
    import torch

    from oracle import cpu_torch_path

    torch.set_num_threads(os.cpu_count() or 1)      # every host thread, as the reference's CPU run would use

    sample = max(1, min(args.cpu_sample, args.batch))
    gen = torch.Generator().manual_seed(1)
    B, H, HV, K, V = sample, shape.heads, shape.value_heads, shape.key_dim, shape.value_dim
    state = torch.randn(B, HV, V, K, generator=gen) * 0.02
    codes, scale = cpu_torch_path.quantize_vblock32(state)
    a_log = torch.rand(HV, generator=gen) * math.log(16.0)
    dt_bias = torch.zeros(HV)
    dec = cpu_torch_path.HostDecoder(codes, scale, a_log, dt_bias, H, window)
    width = 2 * H * K + HV * V
    mixed = torch.randn(window, B, width, generator=gen).to(torch.bfloat16)
    ab = torch.randn(window, 2, B, HV, generator=gen).to(torch.bfloat16)
    threads = torch.get_num_threads()
    dec.step(mixed[0], ab[0, 0], ab[0, 1])          # warm the allocator / thread pool
    dec = cpu_torch_path.HostDecoder(codes, scale, a_log, dt_bias, H, window)
    t0 = time.perf_counter()
    cycles = 0
    while True:                                      # whole cycles, >= CPU_SAMPLE_SECONDS of work
        for t in range(window):
            dec.step(mixed[t], ab[t, 0], ab[t, 1])
        cycles += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= CPU_SAMPLE_SECONDS or cycles >= CPU_MAX_CYCLES:
            break
    us_per_step = elapsed / (cycles * window) * 1e6 * (args.batch / sample)
    scaled = f"; scaled x{args.batch / sample:g} to batch {args.batch}" if sample != args.batch else ""
    host = host_cpu()
    return {
        "value": us_per_step,
        "unit": "us/step",
        "cores": threads,
        "threads": threads,
        "host": host,
        "torch": torch.__version__,
        "kind": "port",
        "sample": (f"{cycles} whole ring cycle(s) ({cycles * window} steps incl. {cycles} flushes) at batch {sample}, "
                   f"same layer shape and cycle as the GPU run, fp32 torch on {threads} host threads, "
                   f"{elapsed:.2f} s{scaled}"),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported (the ReplaySSM path shards "
              "by sequence with no communication; run one process per GPU).", file=sys.stderr)
        return 2

    import torch

    import gdn_replayssm_fp8_kernel as gk
    import gdn_replayssm_synth as synth
    from gdn_replayssm_traffic import LayerShape, bf16_rmw_bytes, cycle_bytes_per_step, reference_traffic

    if not torch.cuda.is_available():
        print("bench.py needs a GPU (the HIP path has no CPU fallback)", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.only:
        stream = torch.cuda.Stream(device)       # default priority
        print(json.dumps({"only": args.only, **run_extras([args.only], device, stream)}), flush=True)
        return 0
    B, L, S = args.batch, args.window, args.sets
    shape = synth.Shape(B)
    traffic_shape = LayerShape(B)
    round_len = S * L
    steps_requested = args.steps
    if args.profile:
        args.steps, args.warmup = 2 * round_len, round_len
        rounds, warm_rounds = 2, 1
    else:
        rounds = max(MIN_TIMED_ROUNDS, math.ceil(args.steps / round_len))
        warm_rounds = max(MIN_WARM_ROUNDS, math.ceil(args.warmup / round_len))
    steps = rounds * round_len
    log(f"[bench] B={B} L={L} sets={S} block_v={args.block_v} phase={args.phase}: "
        f"{rounds} timed rounds of {round_len} steps ({steps} steps), {warm_rounds} warm-up rounds")

    # ---- inputs resident in HBM ----------------------------------------------
    gen = synth.generator(0, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    t0 = time.perf_counter()
    if args.trace:
        # real decode inputs from a capture file (one layer's batch-1 record,
        # replicated over the batch; its steps repeat when fewer than L)
        import gdn_replayssm_capture as cap

        inp = cap.captured_inputs(cap.load_capture(args.trace), B, args.trace_layer, L, device)
        a_log, dt_bias = inp["a_log"], inp["dt_bias"]
        reps = math.ceil(L / inp["mixed_qkv"].shape[1])
        mixed, a_raw, b_raw = (inp[k].repeat(1, reps, 1)[:, :L].contiguous() for k in ("mixed_qkv", "a", "b"))
        state = inp["state"]
    else:
        state = synth.warm_state(shape, 256, gen, device, a_log, dt_bias)
        mixed, a_raw, b_raw = synth.raw_step_inputs(shape, L, gen, device)
    ck = gk.quantize_checkpoint(state, saturation=False)
    del state
    mixed = [mixed[:, t].contiguous() for t in range(L)]
    a_raw = [a_raw[:, t].contiguous() for t in range(L)]
    b_raw = [b_raw[:, t].contiguous() for t in range(L)]
    sets = []
    for _ in range(S):
        sets.append(dict(
            payload=ck.payload.clone(), scale=ck.scale.clone(),
            q_out=torch.zeros(B, shape.heads, 128, dtype=torch.bfloat16, device=device),
            k=torch.zeros(B, L, shape.heads, 128, dtype=torch.bfloat16, device=device),
            v=torch.zeros(B, L, shape.value_heads, 128, dtype=torch.bfloat16, device=device),
            g=torch.zeros(B, L, shape.value_heads, dtype=torch.bfloat16, device=device),
            beta=torch.zeros(B, L, shape.value_heads, dtype=torch.bfloat16, device=device),
            out=torch.empty(B, shape.value_heads, 128, dtype=torch.bfloat16, device=device)))
    # per-step metadata, one variant per position in the cycle
    seq = torch.arange(B, device=device)
    meta = []
    for i in range(L):
        phase = (seq % L) if args.phase == "mixed" else torch.zeros_like(seq)
        fill = ((phase + i) % L + 1).to(torch.int32)
        meta.append(dict(pos=(fill - 1).contiguous(), valid=fill.contiguous(), flush=(fill == L).contiguous()))
    torch.cuda.synchronize()
    log(f"[bench] inputs ready in {time.perf_counter() - t0:.1f} s "
        f"({torch.cuda.memory_allocated() / 2**30:.2f} GiB allocated)")

    def launch(i: int) -> None:
        st = sets[i % S]
        c = (i // S) % L
        m = meta[c]
        gk.gdn_prep_replay_fp8(mixed[c], a_raw[c], b_raw[c], a_log, dt_bias, m["pos"], st["payload"], st["scale"],
                               st["q_out"], st["k"], st["v"], st["g"], st["beta"], m["valid"], m["flush"],
                               block_v=args.block_v, out=st["out"])

    def one_round() -> None:
        for i in range(round_len):
            launch(i)

    # fill every ring once (also compiles nothing: kernels are prebuilt)
    one_round()
    torch.cuda.synchronize()

    stream = torch.cuda.Stream(device)       # default priority
    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            one_round()                       # warm this stream before capture
            stream.synchronize()
            with torch.cuda.graph(graph, stream=stream):
                one_round()
        torch.cuda.synchronize()

    def run_rounds(n: int) -> None:
        with torch.cuda.stream(stream):
            for _ in range(n):
                if graph is not None:
                    graph.replay()
                else:
                    one_round()

    check_waits("set-up")
    run_rounds(warm_rounds)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record(stream)
    run_rounds(rounds)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    check_waits("headline")
    ms_total = start.elapsed_time(end)
    us_step = ms_total * 1e3 / steps
    log(f"[bench] timed {steps} steps: {us_step:.3f} us/step (events), wall {wall * 1e6 / steps:.3f} us/step")

    bytes_step = cycle_bytes_per_step(traffic_shape, L, with_prep=True)
    achieved = bytes_step / (us_step * 1e-6) / 1e9
    result = {
        "metric": METRIC,
        "value": round(us_step, 4),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": steps,
        "steps_requested": steps_requested,
        "warmup": warm_rounds * round_len,
        "ms_per_step": us_step / 1e3,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "storage": "fp8-e4m3fn checkpoint (fp16 vblock32 scales), bf16 ring/q/out",
        "data": (f"capture {args.trace} layer {args.trace_layer} (batch-1 record replicated over the batch)"
                 if args.trace else "synthetic (seeded; BASELINE distributions, 256-step warm-up state)"),
        "config": {
            "workload": (f"full-contract decode step (prep + replay, flush at l=L), one fused launch per step, "
                         f"Qwen3.5-4B GDN layer H=16 HV=32 K=V=128, B={B}, L={L}, cycle-amortised ({args.phase} "
                         f"ring phases), {S} rotating buffer sets"),
            "batch": B, "window": L, "block_v": args.block_v, "buffer_sets": S, "phase": args.phase,
            "hip_graph": graph is not None,
        },
        "seq_per_s": B / (us_step * 1e-6),
        "algorithmic_bytes_per_step": bytes_step,
        "roofline": {
            "bound": "hbm",
            "kernel": KERNEL_NAME.format(gate_f32="true" if a_raw[0].dtype == torch.float32 else "false"),
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(B, L),
        },
        "bytes_vs_bf16_rmw": {
            "bf16_rmw_bytes_per_step": bf16_rmw_bytes(traffic_shape),
            "ratio_cycle_avg": bf16_rmw_bytes(traffic_shape) / bytes_step,
            # the reference's ratio: bf16 bytes / its amortised cycle bytes (one
            # flush per L steps, bench_gdn_replayssm.py:348-353,381)
            "ratio_reference_accounting": bf16_rmw_bytes(traffic_shape)
            / reference_traffic(traffic_shape, L, args.block_v)["amortized_actual"],
        },
        "wall_us_per_step": wall * 1e6 / steps,
    }
    if not args.no_slots and not args.profile:
        slot_us = time_slot_path(args, shape, device, stream, ck, mixed, a_raw, b_raw, a_log, dt_bias, meta, rounds,
                                 warm_rounds)
        result["slot_indexed"] = {
            "us_per_step": round(slot_us, 4),
            "vs_direct": round(slot_us / us_step, 4),
            "layout": f"checkpoint/rings [{B + 1} slots, ...], slot 0 null, batch entry b in slot perm[b] "
                      f"(gdnr_prep_replay_fp8_slots)",
        }
        log(f"[bench] slot-indexed cycle: {slot_us:.3f} us/step ({slot_us / us_step:.3f}x the direct layout)")
    if args.phase == "lockstep" and not args.no_mixed and not args.profile:
        # the same captured cycle with staggered ring phases (sequence b at
        # phase b % L, so every launch flushes B / L sequences): the metadata
        # tensors the graph reads are rewritten in place
        for i in range(L):
            fill = ((seq % L + i) % L + 1).to(torch.int32)
            meta[i]["pos"].copy_(fill - 1)
            meta[i]["valid"].copy_(fill)
            meta[i]["flush"].copy_(fill == L)
        torch.cuda.synchronize()
        run_rounds(warm_rounds)
        torch.cuda.synchronize()
        start.record(stream)
        run_rounds(rounds)
        end.record(stream)
        torch.cuda.synchronize()
        check_waits("mixed phases")
        mixed_us = start.elapsed_time(end) * 1e3 / steps
        result["mixed_phase"] = {
            "us_per_step": round(mixed_us, 4),
            "vs_lockstep": round(mixed_us / us_step, 4),
            "note": "sequence b at ring phase b % L: every launch flushes B/L sequences and lasts as long as their "
                    "rebuild; the headline follows the reference's lockstep cycle",
        }
        log(f"[bench] mixed ring phases: {mixed_us:.3f} us/step ({mixed_us / us_step:.2f}x the lockstep cycle)")
    if not args.no_rmw and not args.profile:
        rmw_us = time_bf16_rmw(shape, device, stream)
        rmw_bytes = bf16_rmw_bytes(traffic_shape)
        result["bf16_rmw"] = {
            "kernel": "rmw_step_kernel<ActBF16, ActBF16>",
            "us_per_step": round(rmw_us, 4),
            "bytes_per_step": rmw_bytes,
            "achieved_GBps": round(rmw_bytes / (rmw_us * 1e-6) / 1e9, 1),
            "frac": round(rmw_bytes / (rmw_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "replayssm_speedup": round(rmw_us / us_step, 3),
        }
        log(f"[bench] bf16 read-modify-write comparator: {rmw_us:.3f} us/step, "
            f"ReplaySSM {rmw_us / us_step:.2f}x faster")
        packed_us = time_bf16_packed(shape, device, stream)
        result["bf16_rmw_packed"] = {
            "kernel": "rmw_step_kernel<ActBF16, ActBF16, 32, PACKED>",
            "contract": "production: raw mixed_qkv, q/k norm + gates in the kernel, slot-indexed state, "
                        "out [B,1,HV,V] (gdnr_bf16_step_packed)",
            "us_per_step": round(packed_us, 4),
            "frac": round(rmw_bytes / (packed_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "replayssm_speedup": round(packed_us / us_step, 3),
        }
        log(f"[bench] production-contract bf16 comparator: {packed_us:.3f} us/step, "
            f"ReplaySSM {packed_us / us_step:.2f}x faster")
    if not args.no_extras and not args.profile:
        extra = run_extras(EXTRAS, device, stream, buffers=[st["payload"] for st in sets])
        result.update(extra)
        result["stream_floor_us"] = extra["stream_floor"]["read_us"]
    if args.cpu_sample > 0 and not args.profile:
        log("[bench] timing the CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(args, traffic_shape, L)
        result["cpu_baseline"]["gpu_speedup"] = result["cpu_baseline"]["value"] / us_step
    else:
        result["cpu_baseline"] = None
    if args.profile:
        calibration_copies(device)
    print(json.dumps(result), flush=True)
    return 0



# ---------------------------------------------------------------------------
# Extra measurements: the reference's kernel benchmark (core kernel over a ring
# cycle, split against fused), BASELINE configs 1 and 3, and the HBM floor.
# ---------------------------------------------------------------------------

GRAPH_MIN_LAUNCHES = 192


def _graph_us(stream, one_round, calls: int, rounds: int = 3, warm: int = 1) -> float:
    """Microseconds per launch: one_round() (`calls` launches) run once
    eagerly, then captured in a HIP graph as many times in a row as makes
    at least GRAPH_MIN_LAUNCHES launches, replayed `warm` + `rounds` times,
    HIP events on the capture stream around the timed replays. (Each replay
    of a graph costs microseconds between its last launch and the next
    replay's first, which a graph of a dozen launches would spread over
    them: the kernel trace then shows the launches shorter than the events
    say.)"""
    import torch

    reps = max(1, math.ceil(GRAPH_MIN_LAUNCHES / calls))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        one_round()
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(reps):
                one_round()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(warm):
            graph.replay()
        start.record(stream)
        for _ in range(rounds):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    check_waits("graph-timed section")
    return start.elapsed_time(end) * 1e3 / (rounds * reps * calls)


def _core_sets(B: int, L: int, S: int, device, seed: int) -> list:
    """S independent (checkpoint, ring) sets at batch B, ring length L: a
    warm FP8 state (64 recurrence steps) and a full ring of prepared tokens
    (q/k L2-normalised, gates from the reference's formulas)."""
    import torch

    import gdn_replayssm_fp8_kernel as gk
    import gdn_replayssm_synth as synth

    shape = synth.Shape(B)
    gen = synth.generator(seed, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    state = synth.warm_state(shape, 64, gen, device, a_log, dt_bias)
    ck = gk.quantize_checkpoint(state, saturation=False)
    del state
    q, k, v, g, beta = synth.ring_inputs(shape, L, gen, device, a_log, dt_bias)
    f32 = dict(dtype=torch.float32, device=device)
    return [dict(payload=ck.payload.clone(), scale=ck.scale.clone(), q=q.clone(), k=k.clone(), v=v.clone(),
                 g=g.clone(), beta=beta.clone(),
                 out=torch.empty(B, shape.value_heads, shape.value_dim, dtype=torch.bfloat16, device=device),
                 tq=torch.empty(B, shape.value_heads, shape.key_dim, **f32),
                 coef=torch.zeros(B, shape.value_heads, L, **f32)) for _ in range(S)]


def _core_launch(st: dict, valid, flush, block_v: int = 128) -> None:
    import gdn_replayssm_fp8_kernel as gk

    gk.gdn_replay_fp8(st["payload"], st["scale"], st["q"], st["k"], st["v"], st["g"], st["beta"], valid, flush,
                      block_v=block_v, out=st["out"])


def time_core_cycles(device, stream, windows=(4, 8, 16), B: int = 64, S: int = 12) -> dict:
    """The reference's kernel benchmark cycle (prototype/bench_gdn_replayssm.py
    :291-330, amortised as :290): the core kernel (gdn_replay_fp8 on prepared
    rings, no prep) at ring fills 1..L-1, then the flush at fill L, over S
    rotating sets; us per step over whole cycles, and the replay at fill L-1
    and the flush alone."""
    import torch

    res = {}
    for L in windows:
        sets = _core_sets(B, L, S, device, seed=300 + L)
        valid = [torch.full((B,), f, dtype=torch.int32, device=device) for f in range(1, L + 1)]
        flush = [torch.full((B,), f == L, dtype=torch.bool, device=device) for f in range(1, L + 1)]

        def cycle():
            for i in range(S * L):
                c = (i // S) % L
                _core_launch(sets[i % S], valid[c], flush[c])

        def at_fill(c):
            def one_round():
                for i in range(S):
                    _core_launch(sets[i], valid[c], flush[c])
            return one_round

        us = _graph_us(stream, cycle, S * L)
        res[f"L{L}"] = {"us_per_step": round(us, 4),
                        "replay_us_at_fill_L-1": round(_graph_us(stream, at_fill(L - 2), S), 4) if L > 1 else None,
                        "flush_us": round(_graph_us(stream, at_fill(L - 1), S), 4)}
        del sets
    res["workload"] = (f"core kernel gdn_replay_fp8, B={B}, H=16 HV=32 K=V=128, block_v=128, fills 1..L-1 then the "
                       f"flush at L, {S} rotating sets, HIP graph")
    return res


def time_config1(device, stream, B: int = 64, L: int = 16, S: int = 12) -> dict:
    """one core-kernel launch at B=64, L=16 with the ring
    fills spread uniformly over 1..16 (sequence b at fill b % 16 + 1; the
    B/16 sequences at 16 flush in the same launch)."""
    import torch

    sets = _core_sets(B, L, S, device, seed=401)
    fill = (torch.arange(B, device=device) % L + 1).to(torch.int32)
    flush = fill == L

    def one_round():
        for i in range(S):
            _core_launch(sets[i], fill, flush)

    us = _graph_us(stream, one_round, S)
    return {"us_per_launch": round(us, 4), "flushing_sequences": int(flush.sum()),
            "workload": f"core kernel, B={B}, L={L}, fills b % {L} + 1 (flush at {L}) in one launch, {S} rotating sets"}


def time_split_vs_fused(device, stream, B: int = 64, L: int = 16, S: int = 12) -> dict:
    """The reference's tiled-against-split comparison (bench_gdn_replayssm.py
    :291-330): the replay at fills 1..L-1 as one fused launch (gdn_replay_fp8)
    and as precompute + apply (gdn_replay_fp8_split), and each cycle with the
    fused flush at fill L."""
    import torch

    import gdn_replayssm_fp8_kernel as gk

    sets = _core_sets(B, L, S, device, seed=501)
    valid = [torch.full((B,), f, dtype=torch.int32, device=device) for f in range(1, L + 1)]
    no_flush = torch.zeros(B, dtype=torch.bool, device=device)
    flush = torch.ones(B, dtype=torch.bool, device=device)

    def fused():
        for i in range(S * (L - 1)):
            _core_launch(sets[i % S], valid[(i // S) % (L - 1)], no_flush)

    def split():
        for i in range(S * (L - 1)):
            st = sets[i % S]
            gk.gdn_replay_fp8_split(st["payload"], st["scale"], st["q"], st["k"], st["v"], st["g"], st["beta"],
                                    valid[(i // S) % (L - 1)], st["tq"], st["coef"], block_v=128, out=st["out"])

    def flush_round():
        for i in range(S):
            _core_launch(sets[i], valid[L - 1], flush)

    fused_us = _graph_us(stream, fused, S * (L - 1))
    split_us = _graph_us(stream, split, S * (L - 1))
    flush_us = _graph_us(stream, flush_round, S)
    return {"fused_replay_us": round(fused_us, 4), "split_replay_us": round(split_us, 4),
            "flush_us": round(flush_us, 4),
            "fused_cycle_us": round(((L - 1) * fused_us + flush_us) / L, 4),
            "split_cycle_us": round(((L - 1) * split_us + flush_us) / L, 4),
            "workload": f"B={B}, L={L}, replay fills 1..{L - 1} (cycle average), block_v=128, {S} rotating sets"}


def _rel_l2(a, b) -> float:
    import torch

    return float(torch.linalg.vector_norm((a - b).double()) / torch.linalg.vector_norm(b.double()))


def config3(device, stream, windows=(4, 16, 64), B: int = 8, steps: int = 4096) -> dict:
    """BASELINE config 3 at B=8, L in {4, 16, 64}: the full-contract step
    (fused prep + replay, flush at fill L) timed over whole ring cycles on
    enough rotating sets to exceed the Infinity Cache; then, untimed, 4096
    steps with fresh seeded inputs beside an fp32 recurrence that consumes
    the ring values the kernel appended (gdn_replayssm_drift.drift_study, the
    reference's drift metric of prototype/qwen35_drift_study.py:355-418), in
    the reference's own input regime and in BASELINE's."""
    import torch

    import gdn_replayssm_fp8_kernel as gk
    import gdn_replayssm_synth as synth
    from gdn_replayssm_drift import drift_study

    res = {}
    shape = synth.Shape(B)
    HV, K, V = shape.value_heads, shape.key_dim, shape.value_dim
    bf = dict(dtype=torch.bfloat16, device=device)
    for L in windows:
        # -- timing
        S = 48
        gen = synth.generator(600 + L, device)
        a_log, dt_bias = synth.gating_params(shape, gen, device)
        state = synth.warm_state(shape, 64, gen, device, a_log, dt_bias)
        ck = gk.quantize_checkpoint(state, saturation=False)
        mixed, a_raw, b_raw = synth.raw_step_inputs(shape, L, gen, device)
        mixed = [mixed[:, t].contiguous() for t in range(L)]
        a_raw = [a_raw[:, t].contiguous() for t in range(L)]
        b_raw = [b_raw[:, t].contiguous() for t in range(L)]
        sets = [dict(payload=ck.payload.clone(), scale=ck.scale.clone(), q_out=torch.zeros(B, shape.heads, K, **bf),
                     k=torch.zeros(B, L, shape.heads, K, **bf), v=torch.zeros(B, L, HV, V, **bf),
                     g=torch.zeros(B, L, HV, **bf), beta=torch.zeros(B, L, HV, **bf),
                     out=torch.empty(B, HV, V, **bf)) for _ in range(S)]
        fills = [torch.full((B,), f, dtype=torch.int32, device=device) for f in range(1, L + 1)]
        poss = [f - 1 for f in fills]  # (formed here: inside the timed cycle they would be a kernel per step)
        flushes = [torch.full((B,), f == L, dtype=torch.bool, device=device) for f in range(1, L + 1)]

        def cycle():
            for i in range(S * L):
                st, c = sets[i % S], (i // S) % L
                gk.gdn_prep_replay_fp8(mixed[c], a_raw[c], b_raw[c], a_log, dt_bias, poss[c], st["payload"],
                                       st["scale"], st["q_out"], st["k"], st["v"], st["g"], st["beta"], fills[c],
                                       flushes[c], block_v=128, out=st["out"])

        us = _graph_us(stream, cycle, S * L, rounds=2)
        del sets, state
        # -- drift (untimed), in the reference's input regime and in BASELINE's
        drift = {}
        for regime, seed in (("reference", 700 + L), ("baseline", 800 + L)):
            d = drift_study(L, device, steps=steps, batch=B, regime=regime, seed=seed)
            drift[regime] = {k: (round(v, 6) if isinstance(v, float) else v) for k, v in d.items()
                             if k not in ("regime", "window")}
        res[f"L{L}"] = {"us_per_step": round(us, 4), "drift": drift}
    res["workload"] = (f"full-contract step (fused prep + replay, flush at L), B={B}, H=16 HV=32 K=V=128, "
                       f"timed over whole cycles on 48 rotating sets; drift over {steps} steps "
                       f"(gdn_replayssm_drift: the reference's metric, qwen35_drift_study.py:355-418) in the "
                       f"reference's make_inputs regime from its 0.02 N(0,1) state and in BASELINE's from zero")
    return res


def stream_floor(device, stream, buffers: list) -> dict:
    """The HBM floor of the checkpoint traffic at the bench's buffer rotation:
    one coalesced pass over each set's codes in turn (gdnr_stream_probe), read
    only (what a replay must read) and read + written back in place (what a
    flush must move); then the same probe swept over buffer sizes from one
    checkpoint's codes (33.5 MB) to 1 GiB, plain and non-temporal loads, read
    and read + write, each size on enough rotating buffers to exceed the
    256 MB Infinity Cache. A line t = t0 + bytes / bw fitted over the sizes a
    decode launch moves (33.5 .. 268 MB) gives the per-launch fixed cost t0
    and the rate bw; the largest sizes run a little slower than that line."""
    import torch

    import gdnr_lib

    def probe(bufs, flags):
        def one_round():
            for buf in bufs:
                gdnr_lib.call("gdnr_stream_probe", [buf], [flags], gdnr_lib.current_stream(device))
        return one_round

    n = len(buffers)
    nbytes = buffers[0].numel() * buffers[0].element_size()
    read_us = _graph_us(stream, probe(buffers, 0), n, rounds=5)
    rw_us = _graph_us(stream, probe(buffers, 1), n, rounds=5)
    res = {"read_us": round(read_us, 4), "read_write_us": round(rw_us, 4), "bytes": nbytes,
           "read_GBps": round(nbytes / (read_us * 1e-6) / 1e9, 1),
           "read_write_GBps": round(2 * nbytes / (rw_us * 1e-6) / 1e9, 1),
           "workload": f"{n} rotating checkpoint code buffers of {nbytes} bytes, one coalesced pass each"}
    modes = {"read": 0, "read_write": 1, "read_nt": 2, "read_write_nt": 3, "read_chunked_nt": 6,
             "read_chunked_tiled_nt": 14}
    sizes = [nbytes << i for i in range(6)]  # 33.5 MB .. 1.07 GB at the headline shape
    sweep = {m: [] for m in modes}
    for size in sizes:
        nbuf = max(2, math.ceil(768 * 2 ** 20 / size))
        bufs = [torch.zeros(size // 16, 16, dtype=torch.uint8, device=device) for _ in range(nbuf)]
        for m, flags in modes.items():
            us = _graph_us(stream, probe(bufs, flags), nbuf, rounds=3)
            moved = size * (2 if flags & 1 else 1)
            sweep[m].append({"bytes": size, "us": round(us, 3), "GBps": round(moved / (us * 1e-6) / 1e9, 1)})
        del bufs
        torch.cuda.empty_cache()
    fits = {}
    for m, pts in sweep.items():
        xs = [p["bytes"] * (2 if modes[m] & 1 else 1) for p in pts if p["bytes"] <= 256 * 2 ** 20]
        ys = [p["us"] for p in pts if p["bytes"] <= 256 * 2 ** 20]
        mx, my = sum(xs) / len(xs), sum(ys) / len(ys)
        slope = sum((x - mx) * (y - my) for x, y in zip(xs, ys)) / sum((x - mx) ** 2 for x in xs)
        fits[m] = {"fixed_us": round(my - slope * mx, 3), "plateau_GBps": round(1e-3 / slope, 1)}
    res["sweep"] = sweep
    res["fit"] = fits
    res["sweep_workload"] = ("gdnr_stream_probe (2048 workgroups of 256 lanes, 16-byte pieces, 4 in flight per lane) "
                             "over rotating buffers of 33.5 MB .. 1.07 GB (>= 768 MiB per rotation); fit over "
                             "33.5 .. 268 MB: t = fixed_us + bytes moved / plateau")
    return res


def run_extras(names, device, stream, buffers=None) -> dict:
    """The extra measurements by name (EXTRAS); buffers: the checkpoint code
    tensors of the headline's sets for the stream floor (fresh ones if None)."""
    import torch

    out = {}
    for name in names:
        t0 = time.perf_counter()
        if name == "core":
            out["core_cycle"] = time_core_cycles(device, stream)
        elif name == "config1":
            out["config1_single_launch"] = time_config1(device, stream)
        elif name == "split":
            out["split_vs_fused"] = time_split_vs_fused(device, stream)
        elif name == "config3":
            out["config3"] = config3(device, stream)
        elif name == "floor":
            if buffers is None:
                buffers = [torch.zeros(64, 32, 128, 128, dtype=torch.uint8, device=device) for _ in range(12)]
            out["stream_floor"] = stream_floor(device, stream, buffers)
        log(f"[bench] extra '{name}' done in {time.perf_counter() - t0:.1f} s")
    return out


def time_slot_path(args, shape, device, stream, ck, mixed, a_raw, b_raw, a_log, dt_bias, meta, rounds,
                   warm_rounds) -> float:
    """The bench cycle again, through the slot-indexed step: every buffer set
    is a cache of B + 1 slots (slot 0 null) holding the batch at a shuffled
    slot permutation, the way vLLM's ssm_state_indices address it. Same
    rounds, graph and event timing as the headline. Returns us per step."""
    import torch

    import gdn_replayssm_fp8_kernel as gk

    B, L, S = args.batch, args.window, args.sets
    gen = torch.Generator(device="cpu")
    gen.manual_seed(3)
    perm = (torch.randperm(B, generator=gen) + 1).to(torch.int32).to(device)
    sets = []
    for _ in range(S):
        payload = torch.zeros(B + 1, *ck.payload.shape[1:], dtype=ck.payload.dtype, device=device)
        scale = torch.ones(B + 1, *ck.scale.shape[1:], dtype=ck.scale.dtype, device=device)
        payload[perm.long()] = ck.payload
        scale[perm.long()] = ck.scale
        sets.append(dict(
            payload=payload, scale=scale,
            q_out=torch.zeros(B, shape.heads, 128, dtype=torch.bfloat16, device=device),
            k=torch.zeros(B + 1, L, shape.heads, 128, dtype=torch.bfloat16, device=device),
            v=torch.zeros(B + 1, L, shape.value_heads, 128, dtype=torch.bfloat16, device=device),
            g=torch.zeros(B + 1, L, shape.value_heads, dtype=torch.bfloat16, device=device),
            beta=torch.zeros(B + 1, L, shape.value_heads, dtype=torch.bfloat16, device=device),
            out=torch.empty(B, shape.value_heads, 128, dtype=torch.bfloat16, device=device)))
    round_len = S * L

    def one_round():
        for i in range(round_len):
            st = sets[i % S]
            c = (i // S) % L
            m = meta[c]
            gk.gdn_prep_replay_fp8(mixed[c], a_raw[c], b_raw[c], a_log, dt_bias, m["pos"], st["payload"],
                                   st["scale"], st["q_out"], st["k"], st["v"], st["g"], st["beta"], m["valid"],
                                   m["flush"], block_v=args.block_v, out=st["out"], state_indices=perm)

    with torch.cuda.stream(stream):
        one_round()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            one_round()
        for _ in range(warm_rounds):
            graph.replay()
        stream.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(rounds):
            graph.replay()
        end.record(stream)
        end.synchronize()
    return start.elapsed_time(end) * 1e3 / (rounds * round_len)


RMW_SETS = 6      # rotating bf16 states: 6 x 67 MB at B=64 exceeds the 256 MB Infinity Cache
RMW_ROUNDS = 50


def time_bf16_rmw(shape, device, stream) -> float:
    """Same-box timing of the comparator the north star names: the bf16
    read-modify-write decode step (gdn_bf16_step, one launch per step) on
    the same layer shape and batch, states rotating over RMW_SETS buffers,
    captured in a HIP graph and timed with HIP events on its stream.
    Returns microseconds per step."""
    import torch

    import gdn_replayssm_fp8_kernel as gk
    import gdn_replayssm_synth as synth

    gen = synth.generator(7, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    q, k, v, g, beta = (x.to(torch.bfloat16) for x in synth.token_inputs(shape, 1, gen, device, a_log, dt_bias))
    q, k, v, g, beta = q[:, 0].contiguous(), k[:, 0].contiguous(), v[:, 0].contiguous(), g[:, 0].contiguous(), \
        beta[:, 0].contiguous()
    states = [0.02 * torch.randn(shape.batch, shape.value_heads, shape.value_dim, shape.key_dim, generator=gen,
                                 device=device).to(torch.bfloat16) for _ in range(RMW_SETS)]

    def one_round():
        for st in states:
            gk.gdn_bf16_step(st, q, k, v, g, beta)

    with torch.cuda.stream(stream):
        one_round()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            one_round()
        for _ in range(5):
            graph.replay()
        stream.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(RMW_ROUNDS):
            graph.replay()
        end.record(stream)
        end.synchronize()
    return start.elapsed_time(end) * 1e3 / (RMW_ROUNDS * RMW_SETS)


def time_bf16_packed(shape, device, stream) -> float:
    """The comparator in the production operator's contract
    (gdn_bf16_step_packed: raw mixed_qkv, q/k norm and gates in the kernel,
    a slot-indexed state, out [B,1,HV,V]) on the same shape and batch: one
    state tensor of RMW_SETS * B + 1 slots, each launch of a round on its own
    B slots (a shuffled order), captured in a HIP graph and timed with HIP
    events on its stream. Returns microseconds per step."""
    import torch

    import gdn_replayssm_fp8_kernel as gk
    import gdn_replayssm_synth as synth

    gen = synth.generator(8, device)
    a_log, dt_bias = synth.gating_params(shape, gen, device)
    mixed, a, b = synth.raw_step_inputs(shape, 1, gen, device)
    mixed, a, b = mixed[:, 0].contiguous(), a[:, 0].contiguous(), b[:, 0].contiguous()
    B = shape.batch
    state = torch.empty(RMW_SETS * B + 1, shape.value_heads, shape.value_dim, shape.key_dim, dtype=torch.bfloat16,
                        device=device)
    state.normal_(0.0, 0.02, generator=gen)
    perm = torch.randperm(RMW_SETS * B, generator=gen, device=device).to(torch.int32) + 1
    slot_sets = [perm[i * B:(i + 1) * B].contiguous() for i in range(RMW_SETS)]
    out = torch.empty(B, 1, shape.value_heads, shape.value_dim, dtype=torch.bfloat16, device=device)

    def one_round():
        for idx in slot_sets:
            gk.gdn_bf16_step_packed(mixed, a, b, a_log, dt_bias, state, idx, out=out)

    with torch.cuda.stream(stream):
        one_round()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            one_round()
        for _ in range(5):
            graph.replay()
        stream.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(RMW_ROUNDS):
            graph.replay()
        end.record(stream)
        end.synchronize()
    return start.elapsed_time(end) * 1e3 / (RMW_ROUNDS * RMW_SETS)


CALIB_BYTES = 64 << 20
CALIB_COPIES = 4


def calibration_copies(device) -> None:
    """The last GPU work of a --profile run: CALIB_COPIES plain copies of
    CALIB_BYTES bytes each (every byte read once and written once), which
    calibrate rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch

    src = torch.randint(0, 256, (CALIB_BYTES,), dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(CALIB_COPIES):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] {CALIB_COPIES} calibration copies of {CALIB_BYTES} bytes done")


if __name__ == "__main__":
    try:
        sys.exit(main())
    except WaitTimeout as e:
        print(f"bench.py: {e}", file=sys.stderr, flush=True)
        print(json.dumps({"metric": METRIC, "value": None, "error": str(e)}), flush=True)
        sys.exit(1)
