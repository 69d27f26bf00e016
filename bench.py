#!/usr/bin/env python3
"""Throughput of the MI355X splitzip Top-16 KV codec (one GPU).

Workloads (seeded synthetic bf16 KV: K = N(0,1) x per-channel scale log-uniform in
[0.1, 10], V = N(0, 0.5); per-layer K/V Top-16 codebooks fit on the same tensor):

* ``llama3-8b-paged`` (default): Llama-3-8B paged KV, 32 layers x (2, 4096 blocks,
  16 tokens, 8 KV heads, 128); 8 requests x 4096 tokens whose block tables are
  disjoint random slices of one seeded permutation of the pool.
* ``llama32-1b-contiguous``: Llama-3.2-1B (16 layers, 8 KV heads, 64), one
  1024-token request on contiguous blocks.
* ``llama3-8b-outliers``: the Llama-3-8B shapes with 1% of the elements replaced by
  outliers of magnitude log-uniform in [1e2, 1e4] (random sign). Top-16 payloads
  overflow their escape capacity and, as the reference connector does, are
  re-encoded as fixed6; the decode is then fixed6 decode + scatter.
* ``llama3-70b-tp8-mixed``: one GPU's share of Llama-3-70B under TP=8 (80 layers,
  1 KV head, 128); 64 requests of log-uniform 128 .. 32768 tokens.
* ``llama3-8b-decode-attention``: fused Top-16 decode + decode attention, Llama-3-8B
  GQA (32 query heads, 8 KV heads, 128), 32 sequences x 8192 tokens per layer, KV
  held only as Top-16 payloads (~0.1% escapes: 0.1% outliers injected), Q = N(0, 1)
  bf16. One step = one decode-attention call per layer over 32 layers.

One codec step = for every layer, gather + encode every request into packed
payloads (one batched launch per codec and layer), then decode + scatter every
payload into a receiver cache through an independent random block table.

The JSON line reports raw bf16 bytes through the round trip per second as
``value``, the encode and decode rates separately, the HBM roofline fraction of
the dominant call from HIP events on the codec's stream, the compression ratio,
and the oracle's multi-threaded CPU codec timed on a bounded sample on this host.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
CALIBRATION_BYTES = 256 << 20
METRIC = "codec encode/decode GB/s of raw bf16 KV (% HBM peak) + compression ratio"
WORKLOADS = ["llama3-8b-paged", "llama32-1b-contiguous", "llama3-8b-outliers",
             "llama3-70b-tp8-mixed", "llama3-8b-decode-attention"]
ATTN_BATCH, ATTN_CONTEXT, ATTN_OUTLIERS = 32, 8192, 0.001
# the benchmark's configurations by index, and the timed steps of the configurations
# that ride along with the headline one
CONFIG_OF = {"llama32-1b-contiguous": "config0", "llama3-8b-paged": "config1",
             "llama3-8b-outliers": "config2", "llama3-70b-tp8-mixed": "config3",
             "llama3-8b-decode-attention": "config4"}
SUB_STEPS = 10
# the fused attention rides along with 40 steps (1,280 calls, ~0.2 s): its per-call
# time keeps falling as the timed region grows (159.2 us over 10 steps, 157.2 over
# 20, 156.1 over 40, measured standalone), so the longer region reports its steady
# state
SUB_STEPS_ATTENTION = 40
# configurations whose ride-along summary also carries the C oracle's CPU rate (the
# small contiguous model and the mixed-context share), each on a bounded sample
SUB_CPU_BASELINE = ("llama32-1b-contiguous", "llama3-70b-tp8-mixed")
SUB_CPU_SECONDS = 4.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=30)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--settle-seconds", type=float, default=0.5,
                   help="after the warmup steps, keep stepping (untimed) until this much "
                        "wall time has passed since the first warmup step")
    p.add_argument("--workload", default="llama3-8b-paged", choices=WORKLOADS)
    p.add_argument("--configs", default="all", choices=["all", "none"],
                   help="also run every other workload (shorter) and report it under "
                        "\"configs\" of the line")
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--cpu-baseline-seconds", type=float, default=10.0,
                   help="codec time of the CPU baseline sample (repeated passes)")
    p.add_argument("--cpu-baseline-layers", type=int, default=2,
                   help="layers of the workload the CPU baseline encodes and decodes")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-steps", type=int, default=0,
                   help="only run this many untimed steps (for rocprofv3), then exit")
    p.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                   help="summarise two rocprofv3 --pmc runs of --profile-steps (FETCH_SIZE, "
                        "then WRITE_SIZE) into HBM bytes per dispatch, print JSON and exit")
    p.add_argument("--counter-summary", metavar="PMC_DIR",
                   help="mean value per dispatch of every counter of a rocprofv3 --pmc run, "
                        "per kernel; print JSON and exit")
    return p.parse_args()


# ---------------------------------------------------------------------------
# HBM traffic from hardware counters

PROFILES = ROOT / "profiles"
# kernels of one call of each direction (the roofline's unit of work)
CALL_KERNELS = {
    "encode": ("top16_encode_tile", "top16_encode_finalize"),
    "decode": ("top16_decode_tile_dir",),
    "attention": ("top16_attention_split", "top16_attention_combine"),
}
# a layer whose Top-16 payloads overflow: the probe encode, then fixed6
CALL_KERNELS_OVERFLOW = {
    "encode": ("top16_encode_tile", "top16_encode_finalize", "palette_encode_tile"),
    "decode": ("palette_decode_tile",),
}


_SLEEP_CYCLES_PER_MS = []


def hold_queue(torch, ms: float = 3.0) -> None:
    """Keeps the GPU busy for about `ms` (a spin kernel) so that the launches queued
    behind it run back to back: per-call timings then measure GPU time, not the
    host's submission latency. Calibrated once with HIP events."""
    if not _SLEEP_CYCLES_PER_MS:
        probe = 1_000_000
        torch.cuda._sleep(probe)  # warm-up
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        torch.cuda._sleep(probe)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS.append(probe / max(e0.elapsed_time(e1), 1e-3))
    torch.cuda._sleep(int(_SLEEP_CYCLES_PER_MS[0] * ms))


def warm_up(torch, step, warmup: int, settle_s: float) -> int:
    """`warmup` untimed steps, then more untimed steps until `settle_s` seconds have
    passed since the first. A few warmup steps on a GPU that was idle are not enough:
    20 timed Llama-3-8B steps after 3 warmup steps read 4.4-4.9 ms per step, and
    3.18 ms after half a second of untimed steps. Returns the steps run."""
    t0 = time.perf_counter()
    done = 0
    while done < warmup or time.perf_counter() - t0 < settle_s:
        step()
        done += 1
        if done >= warmup:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return done


def calibration_copy(torch, device):
    """One plain device copy of CALIBRATION_BYTES (read + write) in the profiled
    process: the reference the FETCH_SIZE / WRITE_SIZE counters are scaled by."""
    src = torch.empty(CALIBRATION_BYTES // 2, dtype=torch.int16, device=device)
    src.fill_(3)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()


def _counter_rows(directory):
    import csv

    rows = []
    for path in sorted(Path(directory).rglob("*counter_collection.csv")):
        with path.open() as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _short_name(kernel_name: str) -> str:
    name = kernel_name.replace("(anonymous namespace)::", "")
    if name.startswith("void "):
        name = name[5:]
    for stop in ("<", "("):
        name = name.split(stop)[0]
    return name.split("::")[-1].strip()


def pmc_summary(fetch_dir, write_dir) -> dict:
    """Average FETCH_SIZE and WRITE_SIZE (KiB per dispatch) of every kernel, each
    scaled by what the same counter reads for the calibration copy (the last device
    copy of the run: CALIBRATION_BYTES read and written): HBM bytes per dispatch =
    1024 * (fetch / f_fetch + write / f_write)."""
    per, calibration = {}, {}
    for counter, directory in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        last = None
        for row in _counter_rows(directory):
            if row["Counter_Name"] != counter:
                continue
            name = _short_name(row["Kernel_Name"])
            value = float(row["Counter_Value"])
            per.setdefault(name, {}).setdefault(counter, []).append(value)
            if "copyBuffer" in name:
                dispatch = int(row["Dispatch_Id"])
                if last is None or dispatch > last[0]:
                    last = (dispatch, value)
        if last is None:
            raise RuntimeError("no calibration copy kernel in the counter runs")
        calibration[counter] = last[1] / (CALIBRATION_BYTES / 1024)
    f_fetch, f_write = calibration["FETCH_SIZE"], calibration["WRITE_SIZE"]
    kernels = {}
    for name, counters in per.items():
        if "FETCH_SIZE" not in counters or "WRITE_SIZE" not in counters:
            continue
        fetch = sum(counters["FETCH_SIZE"]) / len(counters["FETCH_SIZE"])
        write = sum(counters["WRITE_SIZE"]) / len(counters["WRITE_SIZE"])
        kernels[name] = {"dispatches": len(counters["FETCH_SIZE"]),
                         "fetch_KiB": round(fetch, 1), "write_KiB": round(write, 1),
                         "hbm_bytes": int(1024 * (fetch / f_fetch + write / f_write))}
    return {"calibration": {"copy_bytes": CALIBRATION_BYTES, "fetch_factor": round(f_fetch, 4),
                            "write_factor": round(f_write, 4)},
            "kernels": kernels}


def counter_summary(directory) -> dict:
    """Mean value per dispatch of every counter of one rocprofv3 --pmc run, per kernel
    (the SQ counters of a pass, for instance)."""
    sums, dispatches = {}, {}
    for row in _counter_rows(directory):
        name = _short_name(row["Kernel_Name"])
        counter = row["Counter_Name"]
        sums.setdefault(name, {}).setdefault(counter, 0.0)
        sums[name][counter] += float(row["Counter_Value"])
        dispatches.setdefault(name, {}).setdefault(counter, set()).add(row["Dispatch_Id"])
    return {name: {c: round(v / len(dispatches[name][c]), 1) for c, v in counters.items()}
            for name, counters in sums.items()}


def measured_traffic(workload: str, direction: str, overflowed: bool = False):
    """HBM bytes of one call (its kernels' counter bytes) from the committed summary
    profiles/pmc_<workload>.json, or None when there is none."""
    path = PROFILES / f"pmc_{workload}.json"
    if not path.exists():
        return None, None
    summary = json.loads(path.read_text())
    kernels = summary.get("kernels", {})
    names = (CALL_KERNELS_OVERFLOW if overflowed else CALL_KERNELS)[direction]
    if not all(n in kernels for n in names):
        return None, path.name
    return sum(kernels[n]["hbm_bytes"] for n in names), path.name


# ---------------------------------------------------------------------------
# workload

def build_workload(torch, sz, workloads, name: str, seed: int):
    """Layers, batches, codebook tables, buffers and the per-layer codec plan."""
    outliers = 0.0
    if name in {"llama3-8b-paged", "llama3-8b-outliers"}:
        shape, pool = workloads.LLAMA3_8B, 4096
        blocks = [4096 // shape.block_size] * 8
        outliers = 0.01 if name == "llama3-8b-outliers" else 0.0
    elif name == "llama32-1b-contiguous":
        shape, pool = workloads.LLAMA32_1B, 64
        blocks = [1024 // shape.block_size]
    else:
        shape = workloads.LLAMA3_70B_TP8
        tokens = workloads.mixed_context_lengths(torch, 64, 128, 32768, shape.block_size, seed=seed)
        blocks = [t // shape.block_size for t in tokens]
        pool = sum(blocks) + 64
    layers = shape.layers
    if name == "llama32-1b-contiguous":
        send_tables = [list(range(blocks[0]))]
        recv_tables = [list(range(blocks[0]))]
    else:
        send_tables = workloads.random_block_tables(torch, pool, blocks, seed=seed)
        recv_tables = workloads.random_block_tables(torch, pool, blocks, seed=seed + 7919)
    device = torch.device("cuda", 0)
    send = sz.PagedBatch(send_tables, shape.block_words, device)
    recv = sz.PagedBatch(recv_tables, shape.block_words, device)
    w = {"name": name, "shape": shape, "pool": pool, "blocks": blocks, "layers": layers,
         "send": send, "recv": recv, "device": device, "outliers": outliers,
         "kv": [], "tables": [], "books": [], "payloads": [], "plan": []}
    w["workspace"] = send.new_workspace()
    w["dirs"] = []
    for layer in range(layers):
        cache = workloads.make_kv_layer(torch, shape, pool, seed=seed, layer=layer, device=device,
                                        outlier_rate=outliers)
        book = workloads.fit_codebook(torch, cache, send_tables)
        w["kv"].append(cache)
        w["books"].append(book)
        w["tables"].append(sz.top16_tables_for(book, device, torch))
        w["payloads"].append(send.new_payload_buffer())
        # the escape directory the encoder writes next to each layer's payloads
        w["dirs"].append(send.new_directory())
    w["receiver"] = [torch.zeros_like(w["kv"][0]) for _ in range(layers)]
    plan_fallbacks(torch, sz, w)
    return w


def plan_fallbacks(torch, sz, w):
    """Encode every layer once and read the payload headers: payloads whose Top-16
    escapes overflow (byte 0 = 255) are re-encoded as fixed6, as the connector's
    ready step does. The data are seeded, so the plan holds for every step."""
    send, recv = w["send"], w["recv"]
    cache = {}
    for layer in range(w["layers"]):
        encode_top16(sz, w, layer)
        head = payload_headers(torch, w, layer)
        over = tuple(r for r, h in enumerate(head) if h[0] == 255)
        keep = tuple(r for r in range(send.payload_count) if r not in over)
        entry = {"over": over, "keep": keep}
        if over:
            if over not in cache:
                sub_send = sz.PagedBatch([send.block_tables[r] for r in over], send.block_words,
                                         w["device"])
                sub_recv = sz.PagedBatch([recv.block_tables[r] for r in over], recv.block_words,
                                         w["device"])
                offsets, sizes, _ = sub_send.palette_layout(6)
                cache[over] = {"send": sub_send, "recv": sub_recv, "offsets": offsets,
                               "sizes": sizes, "workspace": sub_send.new_palette_workspace(),
                               "presence_first": send.presence_first(over)}
            entry.update(cache[over])
            entry["buffer"] = entry["send"].new_palette_buffer(6)
            # a layer that overflows is encoded as a probe (the connector's choice
            # for a Top-16 attempt after an overflow): presence masks and palette
            # records in the same launches, no escape placement in an overflowed
            # payload, so its fixed6 fallback is one pass
            if "presence" not in w:
                w["presence"] = send.new_presence()
                w["palette_info"] = send.new_palette_info()
            entry["presence"] = w["presence"]
            entry["palette_info"] = w["palette_info"]
            entry["info_first"] = list(over)
        if keep and over:
            key = ("keep", keep)
            if key not in cache:
                cache[key] = sz.PagedBatch([recv.block_tables[r] for r in keep], recv.block_words,
                                           w["device"])
            entry["keep_recv"] = cache[key]
        w["plan"].append(entry)


def encode_top16(sz, w, layer, presence=None, palette_info=None):
    got = sz.encode_top16_paged(w["kv"][layer], w["send"], w["payloads"][layer], w["workspace"],
                                tables=w["tables"][layer], directory=w["dirs"][layer],
                                presence=presence, palette_info=palette_info)
    if got != w["send"].total_encoded_bytes:
        raise RuntimeError(f"layer {layer}: paged encode declined ({got})")


def encode_layer(sz, w, layer):
    """Top-16 for every request; fixed6 for the requests whose Top-16 payload overflows."""
    plan = w["plan"][layer]
    encode_top16(sz, w, layer, plan.get("presence"), plan.get("palette_info"))
    if plan["over"]:
        got = sz.encode_bf16_paged(w["kv"][layer], plan["send"], plan["buffer"],
                                   plan["workspace"], bits=6, palette_info=plan["palette_info"],
                                   info_first=plan["info_first"])
        if got != sum(plan["sizes"]):
            raise RuntimeError(f"layer {layer}: fixed6 fallback encode declined ({got})")


def decode_layer(sz, w, layer):
    send, plan = w["send"], w["plan"][layer]
    if not plan["over"]:
        got = sz.decode_top16_paged(w["payloads"][layer], send.out_offsets, send.encoded_bytes,
                                    w["receiver"][layer], w["recv"], tables=w["tables"][layer],
                                    directory=w["dirs"][layer])
        if got != send.total_raw_bytes:
            raise RuntimeError(f"layer {layer}: paged decode declined ({got})")
        return
    if plan["keep"]:
        keep = plan["keep"]
        got = sz.decode_top16_paged(w["payloads"][layer], [send.out_offsets[r] for r in keep],
                                    [send.encoded_bytes[r] for r in keep], w["receiver"][layer],
                                    plan["keep_recv"], tables=w["tables"][layer])
        if not got:
            raise RuntimeError(f"layer {layer}: paged decode declined")
    got = sz.decode_bf16_paged(plan["buffer"], plan["offsets"], plan["sizes"],
                               w["receiver"][layer], plan["recv"], bits=6)
    if got != plan["send"].total_raw_bytes:
        raise RuntimeError(f"layer {layer}: fixed6 decode declined ({got})")


def final_payload_bytes(w, layer) -> int:
    """Bytes that leave the codec for one layer (what the transport would send)."""
    send, plan = w["send"], w["plan"][layer]
    return sum(send.encoded_bytes[r] for r in plan["keep"]) + sum(plan.get("sizes", []))


def payload_headers(torch, w, layer):
    """The 5-byte headers of a layer's Top-16 payloads (read without copying the
    payloads to the host)."""
    send = w["send"]
    key = "header_index"
    if key not in w:
        w[key] = torch.tensor([o + k for o in send.out_offsets for k in range(5)],
                              dtype=torch.int64, device=w["device"])
    head = w["payloads"][layer].index_select(0, w[key]).cpu().view(-1, 5).tolist()
    return [(h[0], h[1] | (h[2] << 8) | (h[3] << 16) | (h[4] << 24)) for h in head]


def escape_counts(torch, w):
    """Escape entries per layer (from the Top-16 payload headers) and overflowed payloads."""
    total, overflow = 0, 0
    for layer in range(w["layers"]):
        for mode, count in payload_headers(torch, w, layer):
            total += count
            overflow += mode == 255
    return total, overflow


def verify(torch, w):
    """Exact round trip of every layer: receiver blocks == sender blocks."""
    src = torch.tensor([b for t in w["send"].block_tables for b in t], device=w["device"])
    dst = torch.tensor([b for t in w["recv"].block_tables for b in t], device=w["device"])
    for layer in range(w["layers"]):
        a = w["kv"][layer].view(torch.int16).index_select(1, src)
        b = w["receiver"][layer].view(torch.int16).index_select(1, dst)
        if not torch.equal(a, b):
            raise RuntimeError(f"layer {layer}: decoded KV differs from the source")


def time_graph_replay(torch, step, w, steps: int, raw_bytes: int):
    """The same step captured once in a HIP graph and replayed `steps` times (the
    entry points only launch kernels on the current stream, so they capture):
    what the step costs once the host's per-call submission is out of the way,
    which is what bounds the small layers of Llama-3.2-1B. Checked like the eager
    steps."""
    graph = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(graph):
            step()
    except RuntimeError as exc:  # capture not available: report, keep the eager line
        torch.cuda.synchronize()
        return {"skipped": f"graph capture failed: {exc}"[:200]}
    for _ in range(2):
        graph.replay()
    torch.cuda.synchronize()
    verify(torch, w)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_queue(torch)
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    verify(torch, w)
    ms = e0.elapsed_time(e1) / steps
    del graph
    return {"ms_per_step": round(ms, 4), "raw_GBps": round(raw_bytes / (ms * 1e-3) / 1e9, 2)}


def time_histogram(torch, sz, w, reps: int = 10):
    """Per-layer GPU exponent histograms of every request's blocks (the codebook
    fit statistics), checked against torch.bincount on layer 0, then timed with
    HIP events over `reps` calls per layer on the first layers."""
    send = w["send"]
    kv0 = w["kv"][0]
    counts = sz.exponent_histogram_paged(kv0, send)
    ids = send.ids
    for plane in range(2):
        words = kv0[plane].index_select(0, ids).reshape(-1).view(torch.int16).to(torch.int32)
        ref = torch.bincount(torch.bitwise_and(torch.bitwise_right_shift(words, 7), 0xFF),
                             minlength=256)
        if not torch.equal(counts[plane], ref):
            raise RuntimeError("exponent histogram differs from torch.bincount")
    layers = min(w["layers"], 8)
    ws = torch.empty(int(sz.exponent_histogram_workspace_bytes(len(ids), send.block_words)),
                     dtype=torch.uint8, device=w["device"])
    out = torch.empty((2, 256), dtype=torch.int64, device=w["device"])
    stream = torch.cuda.current_stream(w["device"])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_queue(torch)
    e0.record(stream)
    for _ in range(reps):
        for layer in range(layers):
            sz.exponent_histogram_paged(w["kv"][layer], send, workspace=ws, counts=out)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * layers)
    gbps = send.total_raw_bytes / (ms * 1e-3) / 1e9
    return {"ms_per_layer_call": round(ms, 5), "raw_GBps": round(gbps, 2),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)}


def time_writeback(torch, sz, w, reps: int = 10):
    """Codec writeback (payloads moved into the sender's own contiguous block runs)
    per layer call, into a scratch layer so the sender's blocks stay intact for the
    next step; checked byte for byte on layer 0."""
    send = w["send"]
    layout = "each request's own contiguous block run"
    if any(sz.contiguous_run(t) is None for t in send.block_tables):
        # fragmented tables are not written back (as in the reference); the kernel
        # is still measured at this size, request r into consecutive blocks of a
        # scratch layer
        counts = [len(t) for t in send.block_tables]
        if sum(counts) > w["pool"]:
            return None
        tables, at = [], 0
        for c in counts:
            tables.append(list(range(at, at + c)))
            at += c
        send = sz.PagedBatch(tables, send.block_words, w["device"])
        if send.out_offsets != w["send"].out_offsets:
            raise RuntimeError("payload layout differs")
        layout = "scratch layer, request r into blocks of one consecutive run"
    members = list(range(send.payload_count))
    scratch = torch.empty_like(w["kv"][0])
    status = torch.empty(len(members), dtype=torch.uint8, device=w["device"])
    sz.writeback_top16_paged(w["payloads"][0], send, scratch, members, status=status)
    torch.cuda.synchronize()
    # overflowed payloads (header 255) are not written back
    written = [r for r, mode in enumerate(status.cpu().tolist()) if mode == 5]
    moved = sum(send.encoded_bytes[r] for r in written)
    flat = scratch.view(-1).view(torch.uint8)
    plane = 2 * scratch.stride(0)
    for r, (off, size) in enumerate(zip(send.out_offsets, send.encoded_bytes)):
        start, count = sz.contiguous_run(send.block_tables[r])
        seg = 2 * count * send.block_words
        k = 2 * start * scratch.stride(1)
        payload = w["payloads"][0][off:off + size]
        head = min(size, seg)
        if int(payload[0]) == 5 and not (
                torch.equal(flat[k:k + head], payload[:head])
                and torch.equal(flat[plane + k:plane + k + size - head], payload[head:])):
            raise RuntimeError("writeback bytes differ from the payload")
    layers = min(w["layers"], 8)
    stream = torch.cuda.current_stream(w["device"])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_queue(torch)
    e0.record(stream)
    for _ in range(reps):
        for layer in range(layers):
            sz.writeback_top16_paged(w["payloads"][layer], send, scratch, members, status=status)
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / (reps * layers)
    if not written:
        return {"ms_per_layer_call": round(ms, 5), "bytes_moved": 0, "layout": layout,
                "note": "every payload overflowed (header 255): the kernel reads each "
                        "payload's mode byte and moves nothing"}
    gbps = 2 * moved / (ms * 1e-3) / 1e9  # payload read + written once
    return {"ms_per_layer_call": round(ms, 5), "bytes_moved": moved, "hbm_GBps": round(gbps, 2),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "layout": layout}


def time_torchop_sender(torch, sz, w, reps: int = 5, cpu_seconds: float = 3.0):
    """The torch-op sender of requests below 1 MiB (what the reference connector
    sends without Top-16 native decode: sign/magnitude, else the high-byte palette,
    else the nibble planes, else raw words): the workload's sender blocks cut into
    requests of the most whole blocks below 1 MiB, on the first layers. Per layer
    call: the plan (presence + plan kernels), the encode, and the decode + scatter
    into the receiver's blocks, each timed with HIP events over back-to-back calls;
    the host-inclusive sender (plan, host read of the plans, encode) timed by the
    wall clock. Layer 0's round trip is checked word for word. ``cpu_baseline``: the
    oracle's numpy restatement of the reference's torch-op encode on a sample of
    the same requests."""
    import numpy as np

    send, recv = w["send"], w["recv"]
    bw, device = send.block_words, w["device"]
    per = ((1 << 20) - 1) // (4 * bw)   # whole blocks of K and V below 1 MiB
    if per == 0:
        return None
    flat_s = [b for t in send.block_tables for b in t]
    flat_r = [b for t in recv.block_tables for b in t]
    count = len(flat_s) // per
    if count == 0:
        return None
    tables = [flat_s[i * per:(i + 1) * per] for i in range(count)]
    batch = sz.PagedBatch(tables, bw, device)
    rbatch = sz.PagedBatch([flat_r[i * per:(i + 1) * per] for i in range(count)], bw, device)
    layers = min(w["layers"], 8)
    plans, fields, outs, offsets, sizes = [], [], [], [], []
    for layer in range(layers):
        plan = sz.plan_torchop_paged(w["kv"][layer], batch)
        got = sz.read_torchop_plans(plan.cpu().numpy())
        size = [s for _, s in got]
        offs = np.concatenate([[0], np.cumsum(size)[:-1]]).astype(np.int64).tolist()
        out = torch.empty(max(1, sum(size)), dtype=torch.uint8, device=device)
        if sz.encode_torchop_paged(w["kv"][layer], batch, plan, out, offs, size) != sum(size):
            raise RuntimeError("torch-op encode failed")
        plans.append(plan)
        fields.append(got)
        outs.append(out)
        offsets.append(offs)
        sizes.append(size)
    if any(s == 0 for size in sizes for s in size):
        return {"requests": count, "note": "a request no torch-op format compresses (raw "
                                          "passthrough): not timed"}
    raw = batch.total_raw_bytes
    target = w["receiver"][0]
    if sz.decode_torchop_paged(outs[0], offsets[0], sizes[0], target, rbatch) != raw:
        raise RuntimeError("torch-op decode failed")
    ids_s = torch.tensor(flat_s[:count * per], dtype=torch.int64, device=device)
    ids_r = torch.tensor(flat_r[:count * per], dtype=torch.int64, device=device)
    if not torch.equal(target.index_select(1, ids_r).view(torch.int16),
                       w["kv"][0].index_select(1, ids_s).view(torch.int16)):
        raise RuntimeError("torch-op round trip differs from the sender's words")
    stream = torch.cuda.current_stream(device)

    def timed(call):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        # the wrappers' host work per call exceeds the GPU's: a longer hold keeps
        # every queued call back to back
        hold_queue(torch, 30.0)
        e0.record(stream)
        for _ in range(reps):
            for layer in range(layers):
                call(layer)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (reps * layers)

    plan_ms = timed(lambda l: sz.plan_torchop_paged(w["kv"][l], batch, plans=plans[l]))
    enc_ms = timed(lambda l: sz.encode_torchop_paged(w["kv"][l], batch, plans[l], outs[l],
                                                     offsets[l], sizes[l]))
    dec_ms = timed(lambda l: sz.decode_torchop_paged(outs[l], offsets[l], sizes[l],
                                                     w["receiver"][l], rbatch))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        for layer in range(layers):
            plan = sz.plan_torchop_paged(w["kv"][layer], batch, plans=plans[layer])
            size = [s for _, s in sz.read_torchop_plans(plan.cpu().numpy())]
            sz.encode_torchop_paged(w["kv"][layer], batch, plan, outs[layer], offsets[layer],
                                    size)
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) * 1e3 / (reps * layers)
    enc_bytes = sum(sum(size) for size in sizes) / layers
    modes = {}
    for got in fields:
        for mode, _ in got:
            modes[str(mode)] = modes.get(str(mode), 0) + 1

    def frac(nbytes, ms):
        return round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)

    result = {
        "requests": count, "blocks_per_request": per,
        "raw_bytes_per_request": 4 * per * bw, "raw_bytes_per_layer": raw,
        "modes": modes, "encoded_bytes_per_layer": int(enc_bytes),
        "compression_ratio": round(raw / enc_bytes, 5),
        "plan_ms_per_layer_call": round(plan_ms, 5),
        "encode_ms_per_layer_call": round(enc_ms, 5),
        "decode_ms_per_layer_call": round(dec_ms, 5),
        # plan: reads the raw words once; encode: reads them again and writes the
        # payloads; decode: reads the payloads and writes the raw words
        "plan_hbm_frac": frac(raw, plan_ms),
        "encode_hbm_frac": frac(raw + enc_bytes, enc_ms),
        "decode_hbm_frac": frac(raw + enc_bytes, dec_ms),
        # the sender's kernels against one read of the words and one write of the
        # payloads (the reference's choice needs the whole request's statistics
        # before any byte is written, so the words are read twice)
        "sender_gpu_hbm_frac": frac(raw + enc_bytes, plan_ms + enc_ms),
        "sender_host_inclusive_ms_per_layer": round(host_ms, 4),
        "verified": True,
    }
    if cpu_seconds > 0:
        # CPU baseline: the oracle's numpy torch-op encoder on requests of layer 0
        # (test infrastructure, timed as the reported baseline only)
        import oracle

        k = min(count, 16)
        sample = w["kv"][0].index_select(1, ids_s[:k * per]).view(torch.int16).cpu().numpy()
        sample = sample.view(np.uint16).reshape(2, k, per * bw)
        done_bytes, r, t0 = 0, 0, time.perf_counter()
        while time.perf_counter() - t0 < cpu_seconds:
            words = sample[:, r % k].reshape(-1)
            if oracle.encode_torchop(words) is None:
                raise RuntimeError("the oracle declined a request the GPU encoded")
            done_bytes += 2 * words.size
            r += 1
        cpu_s = time.perf_counter() - t0
        result["cpu_baseline"] = {
            "value": round(done_bytes / cpu_s / 1e9, 4), "unit": "GB/s raw bf16 (encode only)",
            "cores": 1, "kind": "port",
            "sample": f"{r} requests of layer 0 ({k} distinct), {round(cpu_s, 1)} s, the "
                      "oracle's numpy torch-op encoder"}
    return result


# ---------------------------------------------------------------------------
# CPU baseline (the oracle's C codec, test infrastructure, timed on this host)

CORES_NOTE = ("threads used = the host's CPU share for this one GPU (OMP_NUM_THREADS, "
              "16 cores of an 8-GPU node); cores_visible = this process's CPU affinity")


def cpu_baseline(torch, w, layers: int, seconds: float = 10.0):
    """The oracle's multi-threaded C codec (gather + canonical Top-16 encode, fixed6
    re-encode of overflowed payloads, then decode + scatter) on this host's cores
    over the first `layers` layers, repeated until about `seconds` of codec time
    have been measured; its payloads are compared with the GPU's on the first pass."""
    import numpy as np

    import oracle

    threads = oracle.default_threads()
    shape, pool, send, recv = w["shape"], w["pool"], w["send"], w["recv"]
    bw = shape.block_words
    sample_layers = min(layers, w["layers"])
    host = [(w["kv"][layer].view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1),
             oracle.top16_tables(w["books"][layer]), w["plan"][layer])
            for layer in range(sample_layers)]
    raw = 0
    t_enc = t_dec = 0.0
    passes = 0
    while passes == 0 or t_enc + t_dec < seconds:
        for layer, (kv, tab, plan) in enumerate(host):
            t0 = time.perf_counter()
            out = oracle.encode_paged_batch(kv, pool * bw, bw, bw, send.block_tables,
                                            send.out_offsets, send.out_bytes, tab, threads=threads)
            fallback = [oracle.palette_encode(oracle.gather(kv, pool * bw, bw, bw,
                                                            send.block_tables[r]), 6)
                        for r in plan["over"]]
            t1 = time.perf_counter()
            target = np.zeros(kv.size, np.uint16)
            if plan["over"]:
                keep = list(plan["keep"])
                if keep:
                    oracle.decode_paged_batch(out, [send.out_offsets[r] for r in keep], target,
                                              pool * bw, bw, bw,
                                              [recv.block_tables[r] for r in keep], tab,
                                              threads=threads)
                for r, payload in zip(plan["over"], fallback):
                    words = oracle.palette_decode(payload, send.count_words[r], 6)
                    oracle.scatter(words, target, len(recv.block_tables[r]), bw, pool * bw, bw,
                                   ids=recv.block_tables[r])
            else:
                oracle.decode_paged_batch(out, send.out_offsets, target, pool * bw, bw, bw,
                                          recv.block_tables, tab, threads=threads)
            t2 = time.perf_counter()
            t_enc += t1 - t0
            t_dec += t2 - t1
            raw += send.total_raw_bytes
            if passes:
                continue
            gpu = w["payloads"][layer].cpu().numpy()
            for r, (off, size) in enumerate(zip(send.out_offsets, send.encoded_bytes)):
                if r in plan["keep"] and bytes(gpu[off:off + size]) != bytes(out[off:off + size]):
                    raise RuntimeError(f"layer {layer}: GPU payload differs from the oracle")
            if plan["over"]:
                gpu6 = plan["buffer"].cpu().numpy()
                for payload, off, size in zip(fallback, plan["offsets"], plan["sizes"]):
                    if bytes(gpu6[off:off + size]) != bytes(payload):
                        raise RuntimeError(
                            f"layer {layer}: GPU fixed6 payload differs from the oracle")
        passes += 1
    sample = (f"{passes} passes over {sample_layers} of {w['layers']} layers: "
              f"{raw / 2**30:.2f} GiB raw bf16 encoded then decoded in "
              f"{t_enc + t_dec:.1f} s of codec time")
    return {
        "value": round(2 * raw / (t_enc + t_dec) / 1e9, 3),
        "unit": "GB/s raw bf16 (encode+decode round trip)",
        "cores": threads,
        "cores_visible": oracle.visible_cores(),
        "cores_note": CORES_NOTE,
        "kind": "port",
        "sample": sample,
        "encode_GBps": round(raw / t_enc / 1e9, 3),
        "decode_GBps": round(raw / t_dec / 1e9, 3),
    }


def cpu_baseline_torch(torch, w, seconds: float = 10.0):
    """``ref-cpu-torch``: the oracle's torch-CPU restatement in the reference's
    op-by-op style (index_select gather, bitwise split, table indexing, strided
    nibble packing, nonzero for escapes; decode by strided unpacking, table
    indexing and index_copy_) on this host's torch threads, over the requests of
    layer 0 in turn until about `seconds` have passed; its payloads are compared
    with the GPU's."""
    import oracle
    from oracle import torch_codec

    send, recv = w["send"], w["recv"]
    kv = w["kv"][0].view(torch.int16).cpu()
    tables = torch.from_numpy(oracle.top16_tables(w["books"][0]).copy())
    target = torch.zeros_like(kv)
    gpu = w["payloads"][0].cpu().numpy()
    raw = 0
    t_enc = t_dec = 0.0
    done = 0
    while done == 0 or t_enc + t_dec < seconds:
        r = done % send.payload_count
        t0 = time.perf_counter()
        payload = torch_codec.encode_paged(kv, [send.block_tables[r]], tables, torch)
        t1 = time.perf_counter()
        torch_codec.decode_paged(payload, target, [recv.block_tables[r]], tables, torch)
        t2 = time.perf_counter()
        t_enc += t1 - t0
        t_dec += t2 - t1
        raw += send.raw_bytes[r]
        if done < send.payload_count:
            off, size = send.out_offsets[r], send.encoded_bytes[r]
            if r in w["plan"][0]["keep"] and bytes(payload[0].numpy()) != bytes(gpu[off:off + size]):
                raise RuntimeError(f"request {r}: torch-CPU payload differs from the GPU's")
        done += 1
    return {
        "value": round(2 * raw / (t_enc + t_dec) / 1e9, 3),
        "unit": "GB/s raw bf16 (encode+decode round trip)",
        "threads": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{done} requests of layer 0 ({raw / 2**30:.2f} GiB raw bf16), "
                  f"{t_enc + t_dec:.1f} s",
        "encode_GBps": round(raw / t_enc / 1e9, 3),
        "decode_GBps": round(raw / t_dec / 1e9, 3),
    }


def python_decoder_rate(w, words: int = 1 << 20):
    """The reference's per-element Python Top-16 decoder (restated in the oracle) on
    a 1 M-word payload: the first blocks of request 0 of layer 0. Reported per
    word, not extrapolated."""
    import numpy as np
    import torch

    import oracle

    send, shape = w["send"], w["shape"]
    blocks = max(1, words // (2 * shape.block_words))
    ids = send.block_tables[0][:blocks]
    kv = w["kv"][0].view(torch.int16).cpu().numpy().view(np.uint16).reshape(2, w["pool"], -1)
    sample = kv[:, ids].reshape(-1)
    tab = oracle.top16_tables(w["books"][0])
    payload = oracle.top16_encode(sample, tab)
    if payload[0] != 5:
        return {"skipped": "the sample overflowed its escape capacity"}
    t0 = time.perf_counter()
    raw = oracle.decode_top16_payload_py(bytes(payload), 2 * sample.size, w["books"][0])
    elapsed = time.perf_counter() - t0
    if raw != sample.tobytes():
        raise RuntimeError("Python decoder result differs")
    return {"words": int(sample.size), "seconds": round(elapsed, 3),
            "ns_per_word": round(elapsed / sample.size * 1e9, 1),
            "raw_GBps": round(2 * sample.size / elapsed / 1e9, 6), "threads": 1}


def time_dropin_fixed6(torch, sz, w, reps: int = 3):
    """The reference connector's per-request fallback for an overflowed request:
    gather by index_select, encode_bf16 (fixed6) into a raw-sized buffer, and
    decode_fixed6 of each payload into the receiver's blocks; for the overflowed
    requests of layer 0, checked against the batched fixed6 payloads and the
    source blocks."""
    plan = w["plan"][0]
    if not plan["over"]:
        return {"skipped": "layer 0 has no overflowed payload"}
    send, recv = w["send"], w["recv"]
    kv = w["kv"][0]
    stream = torch.cuda.current_stream(w["device"])
    members = list(plan["over"])
    ids = [torch.tensor(send.block_tables[r], dtype=torch.int64, device=w["device"])
           for r in members]
    sources = [kv.index_select(1, i) for i in ids]
    outs = [torch.empty(send.raw_bytes[r], dtype=torch.uint8, device=w["device"])
            for r in members]
    target = torch.zeros_like(kv)

    def encode_all(gather: bool):
        for k, r in enumerate(members):
            src = kv.index_select(1, ids[k]) if gather else sources[k]
            if sz.encode_bf16(src, outs[k], bits=6) != plan["sizes"][k]:
                raise RuntimeError("drop-in fixed6 encode declined")

    def decode_all():
        for k, r in enumerate(members):
            got = sz.decode_fixed6(outs[k][:plan["sizes"][k]], target, recv.block_tables[r],
                                   send.raw_bytes[r])
            if got != send.raw_bytes[r]:
                raise RuntimeError("drop-in fixed6 decode declined")

    def timed(fn, *a):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        runs = []
        for _ in range(reps):
            hold_queue(torch)
            e0.record(stream)
            fn(*a)
            e1.record(stream)
            torch.cuda.synchronize()
            runs.append(e0.elapsed_time(e1))
        return statistics.median(runs)

    encode_all(False)
    decode_all()
    torch.cuda.synchronize()
    for k, r in enumerate(members):
        off, size = plan["offsets"][k], plan["sizes"][k]
        if not torch.equal(outs[k][:size], plan["buffer"][off:off + size]):
            raise RuntimeError("drop-in fixed6 payload differs from the batched one")
        dst = torch.tensor(recv.block_tables[r], dtype=torch.int64, device=w["device"])
        if not torch.equal(kv.view(torch.int16).index_select(1, ids[k]),
                           target.view(torch.int16).index_select(1, dst)):
            raise RuntimeError("drop-in fixed6 round trip differs")
    raw = sum(send.raw_bytes[r] for r in members)
    ms_gather_enc = timed(encode_all, True)
    ms_enc = timed(encode_all, False)
    ms_dec = timed(decode_all)

    def rate(ms):
        return round(raw / (ms * 1e-3) / 1e9, 2)

    return {
        "requests": len(members),
        "gather_encode_ms_per_request": round(ms_gather_enc / len(members), 5),
        "encode_ms_per_request": round(ms_enc / len(members), 5),
        "encode_raw_GBps": rate(ms_enc),
        "decode_ms_per_request": round(ms_dec / len(members), 5),
        "decode_raw_GBps": rate(ms_dec),
        "layout": "payload at the start of a raw-sized uint8 buffer (low bytes 65 bytes in); "
                  "gather by index_select as the reference connector",
    }


def time_dropin(torch, sz, w, reps: int = 3):
    """The reference-ABI per-request path an unchanged reference connector takes:
    index_select gather of a request's blocks into a packed copy, encode_top16 into
    a raw-sized byte buffer (payload at its start, so the body section is 5 bytes
    off 16-byte alignment), and decode_top16 of each payload into the receiver's
    blocks; for the 8 requests of layer 0, checked against the batched payloads.
    Also the encode at the ABI's minimum capacity (align4(E) + 8 bytes)."""
    send, recv = w["send"], w["recv"]
    kv, books = w["kv"][0], w["books"][0]
    if w["plan"][0]["over"]:
        return {"skipped": "layer 0 has overflowed payloads"}
    stream = torch.cuda.current_stream(w["device"])
    ids = [torch.tensor(t, dtype=torch.int64, device=w["device"]) for t in send.block_tables]
    outs = [torch.empty(n, dtype=torch.uint8, device=w["device"]) for n in send.raw_bytes]
    target = torch.zeros_like(kv)

    def encode_all(gather: bool, sources=None):
        for r in range(send.payload_count):
            src = kv.index_select(1, ids[r]) if gather else sources[r]
            if sz.encode_top16(src, outs[r], -1, codebooks=books) != send.encoded_bytes[r]:
                raise RuntimeError("drop-in encode declined")

    def decode_all():
        for r in range(send.payload_count):
            got = sz.decode_top16(outs[r][:send.encoded_bytes[r]], target, recv.block_tables[r],
                                  send.raw_bytes[r], -1, codebooks=books)
            if got != send.raw_bytes[r]:
                raise RuntimeError("drop-in decode declined")

    sources = [kv.index_select(1, i) for i in ids]

    def timed(fn, *a):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = []
        for _ in range(reps):
            hold_queue(torch)
            e0.record(stream)
            fn(*a)
            e1.record(stream)
            torch.cuda.synchronize()
            best.append(e0.elapsed_time(e1))
        return statistics.median(best)

    encode_all(False, sources)
    decode_all()
    torch.cuda.synchronize()
    for r in range(send.payload_count):
        batched = w["payloads"][0][send.out_offsets[r]:send.out_offsets[r] + send.encoded_bytes[r]]
        if not torch.equal(outs[r][:send.encoded_bytes[r]], batched):
            raise RuntimeError("drop-in payload differs from the batched one")
    src_ids = torch.cat(ids)
    dst_ids = torch.tensor([b for t in recv.block_tables for b in t], device=w["device"])
    if not torch.equal(kv.view(torch.int16).index_select(1, src_ids),
                       target.view(torch.int16).index_select(1, dst_ids)):
        raise RuntimeError("drop-in round trip differs")
    raw = send.total_raw_bytes
    ms_gather_enc = timed(encode_all, True)
    ms_enc = timed(encode_all, False, sources)
    ms_dec = timed(decode_all)
    # minimum capacity: no room for the parallel tiles' workspace past the payload
    r0 = 0
    e = send.encoded_bytes[r0]
    tight = torch.empty(((e + 3) & ~3) + 8, dtype=torch.uint8, device=w["device"])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    sz.encode_top16(sources[r0], tight, -1, codebooks=books)
    hold_queue(torch)
    e0.record(stream)
    sz.encode_top16(sources[r0], tight, -1, codebooks=books)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_tight = e0.elapsed_time(e1)
    if not torch.equal(tight[:e], outs[r0][:e]):
        raise RuntimeError("minimum-capacity payload differs")

    def rate(ms, nbytes):
        return round(nbytes / (ms * 1e-3) / 1e9, 2)

    return {
        "requests": send.payload_count,
        "gather_encode_ms_per_request": round(ms_gather_enc / send.payload_count, 5),
        "gather_encode_raw_GBps": rate(ms_gather_enc, raw),
        "encode_ms_per_request": round(ms_enc / send.payload_count, 5),
        "encode_raw_GBps": rate(ms_enc, raw),
        "decode_ms_per_request": round(ms_dec / send.payload_count, 5),
        "decode_raw_GBps": rate(ms_dec, raw),
        "min_capacity_encode_ms": round(ms_tight, 5),
        "min_capacity_encode_raw_GBps": rate(ms_tight, send.raw_bytes[r0]),
        "layout": "payload at the start of a raw-sized uint8 buffer (body 5 bytes past "
                  "16-byte alignment); gather by index_select as the reference connector",
    }


def time_connector(torch, sz, w, layers: int = 8, rounds: int = 3):
    """The connector's codec hooks over whole layers, as a serving engine calls them:
    save_kv_layer (batched Top-16 encode with its escape directory, the payloads'
    device-to-host copy on the copy stream into the pinned pool), ready (waits for
    the copies and makes the fallback payloads of overflowed requests), then
    load_kv_layer_batch on the receiver (one pinned host-to-device copy, the escape
    directory built on the host, one decode launch per payload mode). Wall-clock
    per layer with the host's work included (PCIe-bound: the payloads cross it
    twice), the host time of each hook and the bytes copied to the host. Layer 0's
    restore is checked against the sender's blocks.

    Where layers overflow (the 1 % outlier workload) the first save of each layer
    tries Top-16 on every request and falls back to fixed6 in ready; the later
    saves follow the per-layer backoff (one probe request per layer, whose payload
    is copied only if its mode byte shows it fits, the rest fixed6). The two are
    summarised separately."""
    from unchainkv_amd.connector import CodecConfig, SplitzipLayerCodec

    layers = min(layers, w["layers"])
    send, recv = w["send"], w["recv"]
    codec = SplitzipLayerCodec(CodecConfig(top16=True, writeback=False),
                               codebooks={layer: w["books"][layer] for layer in range(layers)})

    def one(layer):
        t0 = time.perf_counter()
        pending = codec.save_kv_layer(layer, w["kv"][layer], send.block_tables)
        t1 = time.perf_counter()
        payloads = codec.ready(pending)
        t2 = time.perf_counter()
        requests = [(rt, p.view, p.metadata(layer, send.block_words))
                    for rt, p in zip(recv.block_tables, payloads)]
        t3 = time.perf_counter()
        got = codec.load_kv_layer_batch(layer, w["receiver"][layer], requests)
        t4 = time.perf_counter()
        torch.cuda.synchronize()
        t5 = time.perf_counter()
        codec.release(pending)
        if got != [(len(t), 4 * len(t) * send.block_words) for t in send.block_tables]:
            raise RuntimeError(f"layer {layer}: connector restore declined ({got})")
        modes = sorted({int(p.view[0]) for p in payloads})
        return (t1 - t0, t2 - t1, t4 - t3, t5 - t0, sum(p.encoded_bytes for p in payloads),
                pending.d2h_bytes, modes)

    def summary(rows):
        med = [statistics.median(r[k] for r in rows) * 1e3 for k in range(4)]
        return {"save_host_ms": round(med[0], 3), "ready_ms": round(med[1], 3),
                "load_host_ms": round(med[2], 3), "wall_ms_per_layer": round(med[3], 3),
                "raw_GBps_end_to_end": round(send.total_raw_bytes / (med[3] * 1e-3) / 1e9, 2),
                "payload_bytes": rows[-1][4],
                "d2h_bytes_per_layer": int(statistics.median(r[5] for r in rows)),
                "payload_modes": sorted({m for r in rows for m in r[6]})}

    first = [one(0)]
    src = torch.tensor([b for t in send.block_tables for b in t], device=w["device"])
    dst = torch.tensor([b for t in recv.block_tables for b in t], device=w["device"])
    if not torch.equal(w["kv"][0].view(torch.int16)[:, src],
                       w["receiver"][0].view(torch.int16)[:, dst]):
        raise RuntimeError("connector round trip differs from the sender's blocks")
    overflow = any(p["over"] for p in w["plan"][:layers])
    first += [one(layer) for layer in range(1, layers)]
    later = [one(layer) for _ in range(rounds - 1) for layer in range(layers)]
    result = {"layers": layers, "raw_bytes_per_layer": send.total_raw_bytes,
              "note": "PCIe-inclusive: the payloads go to host memory and back"}
    if not overflow:
        result.update(summary(first + later))
        return result
    result["first_save"] = summary(first)
    result["first_save"]["what"] = ("every request tries Top-16 and overflows; ready "
                                    "re-encodes them as fixed6 (staged on the copy stream)")
    result["backoff"] = summary(later)
    result["backoff"]["what"] = ("per layer one probe request (its Top-16 payload crosses "
                                 "PCIe only if it fits), the others fixed6")
    return result


def time_overlap(torch, sz, w, repeats: int = 7):
    """Encode + device-to-host copy of a layer's payloads against the model's
    attention, in the modes of the reference's scripts/bench_codec_attention.py:
    attention alone, encode alone, copy alone, fully serial (the copy on the
    forward stream: attention waits for it), serial pipeline (encode on the forward
    stream, copy on a copy stream beside the attention: what the connector does)
    and concurrent pipeline (encode and copy on side streams). The attention is
    causal prefill over the layer's 8 x 4096 tokens (32 query heads, 8 KV heads,
    flash kernel); all streams at the default priority."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    send, shape = w["send"], w["shape"]
    device = w["device"]
    g = torch.Generator(device=device)
    g.manual_seed(5)
    reqs, tokens = send.payload_count, len(send.block_tables[0]) * shape.block_size
    q = torch.randn((reqs, 4 * shape.kv_heads, tokens, shape.head_dim), generator=g,
                    device=device).to(torch.bfloat16)
    k = torch.randn((reqs, shape.kv_heads, tokens, shape.head_dim), generator=g,
                    device=device).to(torch.bfloat16)
    v = torch.randn_like(k)

    def attention():
        with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
            return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                                    enable_gqa=True)
    try:
        attention()
        torch.cuda.synchronize()
    except Exception as exc:  # noqa: BLE001 - no flash kernel for this build: report it
        return {"skipped": f"flash attention unavailable: {exc}"[:200]}
    main = torch.cuda.current_stream(device)
    codec = torch.cuda.Stream(device=device)
    copy = torch.cuda.Stream(device=device)
    payloads = w["payloads"][0]
    host = torch.empty(payloads.numel(), dtype=torch.uint8, pin_memory=True)

    def encode():
        encode_top16(sz, w, 0)

    def run(mode):
        ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
        start = ev()
        start.record(main)
        ends = {}
        enc_end = None
        if mode in ("encode_only", "fully_serial", "serial_pipeline"):
            encode()
            enc_end = ev()
            enc_end.record(main)
            ends["encode"] = enc_end
        elif mode == "concurrent_pipeline":
            codec.wait_event(start)
            with torch.cuda.stream(codec):
                encode()
                enc_end = ev()
                enc_end.record(codec)
            ends["encode"] = enc_end
        if mode in ("d2h_only", "fully_serial", "serial_pipeline", "concurrent_pipeline"):
            stream = main if mode == "fully_serial" else copy
            stream.wait_event(enc_end if enc_end is not None else start)
            with torch.cuda.stream(stream):
                host.copy_(payloads, non_blocking=True)
                end = ev()
                end.record(stream)
            ends["d2h"] = end
        if mode in ("attention_only", "fully_serial", "serial_pipeline", "concurrent_pipeline"):
            attention()
            end = ev()
            end.record(main)
            ends["attention"] = end
        for e in ends.values():
            e.synchronize()
        return max(start.elapsed_time(e) for e in ends.values())

    modes = ("attention_only", "encode_only", "d2h_only", "fully_serial", "serial_pipeline",
             "concurrent_pipeline")
    for m in modes:
        run(m)
    samples = {m: [] for m in modes}
    for rep in range(repeats):
        for m in modes[rep % len(modes):] + modes[:rep % len(modes)]:
            samples[m].append(run(m))
    torch.cuda.synchronize()
    if not torch.equal(host, payloads.cpu()):
        raise RuntimeError("staged payload bytes differ")
    out = {m: round(statistics.median(v), 4) for m, v in samples.items()}
    hidden = out["fully_serial"] - out["serial_pipeline"]
    return {"wall_ms_p50": out, "payload_bytes": int(send.total_encoded_bytes),
            "copy_hidden_ms": round(hidden, 4),
            "attention": f"causal flash SDPA, {reqs} x {tokens} tokens, "
                         f"{4 * shape.kv_heads} q heads / {shape.kv_heads} kv heads x "
                         f"{shape.head_dim}, bf16"}


# ---------------------------------------------------------------------------
# fused decode attention workload

def build_attention(torch, sz, workloads, seed: int):
    """32 layers of Llama-3-8B KV for 32 sequences x 8192 tokens, kept only as
    Top-16 payloads (the raw cache of a layer is freed after its encode)."""
    shape = workloads.LLAMA3_8B
    blocks = ATTN_CONTEXT // shape.block_size
    pool = ATTN_BATCH * blocks
    tables = workloads.random_block_tables(torch, pool, [blocks] * ATTN_BATCH, seed=seed)
    device = torch.device("cuda", 0)
    batch = sz.PagedBatch(tables, shape.block_words, device)
    ws = batch.new_workspace()
    w = {"shape": shape, "batch": batch, "device": device, "layers": shape.layers,
         "payloads": [], "tables": [], "books": [], "q": [], "out": []}
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    q_heads = 4 * shape.kv_heads
    for layer in range(shape.layers):
        kv = workloads.make_kv_layer(torch, shape, pool, seed=seed, layer=layer, device=device,
                                     outlier_rate=ATTN_OUTLIERS)
        book = workloads.fit_codebook(torch, kv, tables)
        tab = sz.top16_tables_for(book, device, torch)
        payload = batch.new_payload_buffer()
        if sz.encode_top16_paged(kv, batch, payload, ws, tables=tab) != batch.total_encoded_bytes:
            raise RuntimeError(f"layer {layer}: encode declined")
        if layer in (0, shape.layers - 1):
            back = torch.zeros_like(kv)
            sz.decode_top16_paged(payload, batch.out_offsets, batch.encoded_bytes, back, batch,
                                  tables=tab)
            if not torch.equal(back.view(torch.int16), kv.view(torch.int16)):
                raise RuntimeError(f"layer {layer}: Top-16 round trip differs")
            del back
        del kv
        w["payloads"].append(payload)
        w["tables"].append(tab)
        w["books"].append(book)
        w["q"].append(torch.randn((ATTN_BATCH, q_heads, shape.head_dim), generator=g,
                                  device=device).to(torch.bfloat16))
        w["out"].append(torch.empty((ATTN_BATCH, q_heads, shape.head_dim), dtype=torch.bfloat16,
                                    device=device))
    need = sz.decode_attention_workspace_bytes(ATTN_BATCH, shape.kv_heads, ATTN_CONTEXT)
    w["attn_ws"] = torch.empty(need, dtype=torch.uint8, device=device)
    return w


def attend_layer(sz, w, layer):
    got = sz.decode_attention_top16(w["q"][layer], w["payloads"][layer], w["batch"].out_offsets,
                                    [ATTN_CONTEXT] * ATTN_BATCH, w["shape"].kv_heads,
                                    tables=w["tables"][layer], out=w["out"][layer],
                                    workspace=w["attn_ws"])
    if got is None:
        raise RuntimeError(f"layer {layer}: decode attention declined")


def attention_reference(torch, sz, w, layer):
    """Decode-then-attend on the GPU: the codec's decoder restores the bf16 KV, then
    float32 attention (contiguous operands)."""
    shape, batch = w["shape"], w["batch"]
    hkv, d = shape.kv_heads, shape.head_dim
    blocks = ATTN_CONTEXT // shape.block_size
    kv = torch.zeros((2, ATTN_BATCH * blocks, shape.block_size, hkv, d), dtype=torch.bfloat16,
                     device=w["device"])
    sz.decode_top16_paged(w["payloads"][layer], batch.out_offsets, batch.encoded_bytes, kv, batch,
                          tables=w["tables"][layer])
    ids = torch.tensor([b for t in batch.block_tables for b in t], device=w["device"])
    k = kv[0].index_select(0, ids).reshape(ATTN_BATCH, ATTN_CONTEXT, hkv, d).float()
    v = kv[1].index_select(0, ids).reshape(ATTN_BATCH, ATTN_CONTEXT, hkv, d).float()
    del kv
    qf = w["q"][layer].float().reshape(ATTN_BATCH, hkv, 4, d)
    s = torch.matmul(qf, k.permute(0, 2, 3, 1).contiguous()) / d ** 0.5
    p = torch.softmax(s, dim=-1)
    out = torch.matmul(p, v.permute(0, 2, 1, 3).contiguous())
    return out.reshape(ATTN_BATCH, 4 * hkv, d)


def verify_attention(torch, sz, w, layer):
    ref = attention_reference(torch, sz, w, layer)
    got = w["out"][layer].float()
    err = (got - ref).abs().amax(dim=-1) / ref.abs().amax(dim=-1).clamp_min(1e-6)
    worst = float(err.max())
    if not worst <= 1e-2:
        raise RuntimeError(f"layer {layer}: fused attention off by {worst:.3g} relative")
    return worst


def attention_escapes(torch, w):
    batch, total = w["batch"], 0
    for layer in range(w["layers"]):
        host = w["payloads"][layer].cpu()
        for off in batch.out_offsets:
            head = bytes(host[off:off + 5].tolist())
            if head[0] != 5:
                raise RuntimeError(f"layer {layer}: a payload overflowed its escape capacity")
            total += int.from_bytes(head[1:5], "little")
    return total


def cpu_attention_baseline(torch, w, ref_layer_out):
    """The oracle's C decoder (one payload per thread) then numpy float32 attention,
    over every sequence of layer 0, on this host's cores; checked against the GPU."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    shape, batch = w["shape"], w["batch"]
    hkv, d = shape.kv_heads, shape.head_dim
    threads = oracle.default_threads()
    host = w["payloads"][0].cpu().numpy()
    tab = oracle.top16_tables(w["books"][0])
    q = w["q"][0].float().cpu().numpy()
    n = 2 * ATTN_CONTEXT * hkv * d

    def one(r):
        off = batch.out_offsets[r]
        words = oracle.top16_decode(host[off:off + batch.encoded_bytes[r]], n, tab)
        kv = (words.astype(np.uint32) << 16).view(np.float32).reshape(2, ATTN_CONTEXT, hkv, d)
        k = kv[0].transpose(1, 0, 2)                       # (h, t, d)
        v = kv[1].transpose(1, 0, 2)
        qg = q[r].reshape(hkv, 4, d)
        sc = np.matmul(k, qg.transpose(0, 2, 1)) / np.sqrt(d)   # (h, t, 4)
        sc = np.exp(sc - sc.max(axis=1, keepdims=True))
        p = sc / sc.sum(axis=1, keepdims=True)
        return np.matmul(p.transpose(0, 2, 1), v).reshape(4 * hkv, d)

    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        outs = list(pool.map(one, range(ATTN_BATCH)))
    elapsed = time.perf_counter() - t0
    got = np.stack(outs)
    ref = ref_layer_out.float().cpu().numpy()
    rel = np.abs(got - ref).max(axis=-1) / np.maximum(np.abs(ref).max(axis=-1), 1e-6)
    if not rel.max() <= 1e-2:
        raise RuntimeError("CPU decode-then-attend disagrees with the GPU output")
    raw = 2 * n * ATTN_BATCH
    return {
        "value": round(raw / elapsed / 1e9, 3),
        "unit": "GB/s raw bf16 KV attended (decode-then-attend)",
        "cores": threads,
        "cores_visible": oracle.visible_cores(),
        "cores_note": CORES_NOTE,
        "kind": "port",
        "sample": f"layer 0 of {w['layers']}: {ATTN_BATCH} sequences x {ATTN_CONTEXT} tokens "
                  f"({raw / 2**30:.2f} GiB raw bf16)",
    }


def run_attention(args, torch, sz, workloads, headline: bool = True):
    """Fused decode-attention workload; the JSON object of its run."""
    w = build_attention(torch, sz, workloads, args.seed)
    layers, batch, shape = w["layers"], w["batch"], w["shape"]
    stream = torch.cuda.current_stream(w["device"])

    def step():
        for layer in range(layers):
            attend_layer(sz, w, layer)

    if args.profile_steps:
        for _ in range(args.profile_steps):
            step()
        torch.cuda.synchronize()
        verify_attention(torch, sz, w, 0)
        calibration_copy(torch, w["device"])
        return {"profile_steps": args.profile_steps, "workload": "llama3-8b-decode-attention",
                "calibration_copy_bytes": CALIBRATION_BYTES}

    steps = args.steps if headline else SUB_STEPS_ATTENTION
    warm_up(torch, step, args.warmup if headline else 2, args.settle_seconds)
    worst = max(verify_attention(torch, sz, w, layer) for layer in (0, layers - 1))

    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / steps
    call_ms = ms_per_step / layers

    # the decode half of decode-then-attend, for comparison: the codec's decoder
    # writing one layer's bf16 KV (1 GiB) per call
    receiver = torch.empty((2, ATTN_BATCH * ATTN_CONTEXT // shape.block_size, shape.block_size,
                            shape.kv_heads, shape.head_dim), dtype=torch.bfloat16,
                           device=w["device"])
    for layer in range(2):
        sz.decode_top16_paged(w["payloads"][layer], batch.out_offsets, batch.encoded_bytes,
                              receiver, batch, tables=w["tables"][layer])
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    hold_queue(torch)
    e0.record(stream)
    for layer in range(layers):
        sz.decode_top16_paged(w["payloads"][layer], batch.out_offsets, batch.encoded_bytes,
                              receiver, batch, tables=w["tables"][layer])
    e1.record(stream)
    torch.cuda.synchronize()
    decode_only_ms = e0.elapsed_time(e1) / layers
    del receiver

    escapes = attention_escapes(torch, w) / layers
    from unchainkv_amd import codec_format

    cap_bytes = sum(5 * codec_format.top16_escape_capacity(n) for n in batch.count_words)
    used_payload = batch.total_encoded_bytes - cap_bytes + 5 * escapes
    q_heads = 4 * shape.kv_heads
    partial = w["attn_ws"].numel()  # the split partials (m, l, acc[128]) in float32
    qo = 2 * ATTN_BATCH * q_heads * shape.head_dim * 2
    # algorithmic HBM bytes per call: packed K and V (used escape entries only), Q
    # and out, the split partials written and read back once
    b_call = used_payload + qo + 2 * partial
    achieved = b_call / (call_ms * 1e-3) / 1e9
    raw_layer = batch.total_raw_bytes
    flops = 2 * 2 * ATTN_BATCH * q_heads * ATTN_CONTEXT * shape.head_dim
    traffic, traffic_source = measured_traffic("llama3-8b-decode-attention", "attention")
    result = {
        "metric": METRIC,
        "value": round(raw_layer * layers / (ms_per_step * 1e-3) / 1e9, 2),
        "unit": "GB/s raw bf16 KV attended (fused Top-16 decode + decode attention)",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 MFMA, f32 softmax/accumulate (codec: u16 bit patterns)",
        "data": (f"synthetic seeded (seed {args.seed}); K=N(0,1)*logU[0.1,10] per channel, "
                 f"V=N(0,0.5), {ATTN_OUTLIERS:.1%} outliers +-logU[1e2,1e4]; Q=N(0,1) bf16"),
        "config": {
            "workload": "llama3-8b-decode-attention",
            "layers": layers,
            "batch": ATTN_BATCH,
            "context": ATTN_CONTEXT,
            "q_heads": q_heads,
            "kv_heads": shape.kv_heads,
            "head_dim": shape.head_dim,
            "block_size": shape.block_size,
            "raw_bytes_per_step": raw_layer * layers,
        },
        "ms_per_layer_call": round(call_ms, 5),
        "context_splits": partial // (ATTN_BATCH * shape.kv_heads * 4 * (shape.head_dim + 2) * 4),
        "escape_fraction": round(escapes / (raw_layer / 2), 6),
        "compression_ratio": round(raw_layer / used_payload, 5),
        "max_rel_error_vs_decode_then_attend": round(worst, 6),
        "decode_only_ms_per_layer": round(decode_only_ms, 5),
        "mfma_TFLOPs": round(flops / (call_ms * 1e-3) / 1e12, 2),
        "roofline": {
            "kernel": "top16_attention_split+top16_attention_combine",
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes_per_call": int(b_call),
            "ms_per_call": round(call_ms, 5),
        },
        "wall_s_timed": round(wall, 3),
        "verified": True,
    }
    if headline and not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_attention_baseline(torch, w, w["out"][0])
    return result


# ---------------------------------------------------------------------------
# main

def run_codec(args, torch, sz, workloads, name: str, headline: bool = True):
    """One codec workload (encode + decode of every layer per step); the JSON object
    of its run. The headline run adds the histogram, writeback, graph replay,
    drop-in, overlap and CPU-baseline legs; the ride-along runs of SUB_CPU_BASELINE
    add the C oracle's CPU rate on a short sample."""
    from unchainkv_amd import codec_format

    w = build_workload(torch, sz, workloads, name, args.seed)
    layers = w["layers"]
    stream = torch.cuda.current_stream(w["device"])

    def step(events=None):
        if events:
            events[0].record(stream)
        for layer in range(layers):
            encode_layer(sz, w, layer)
        if events:
            events[1].record(stream)
        for layer in range(layers):
            decode_layer(sz, w, layer)
        if events:
            events[2].record(stream)

    if args.profile_steps:
        for _ in range(args.profile_steps):
            step()
        torch.cuda.synchronize()
        verify(torch, w)
        time_writeback(torch, sz, w, reps=1)
        if name == "llama3-8b-paged":
            time_torchop_sender(torch, sz, w, reps=1, cpu_seconds=0.0)
        calibration_copy(torch, w["device"])
        return {"profile_steps": args.profile_steps, "workload": name,
                "calibration_copy_bytes": CALIBRATION_BYTES}

    steps = args.steps if headline else SUB_STEPS
    warm_up(torch, step, args.warmup if headline else 2, args.settle_seconds)
    verify(torch, w)

    # timed region: exactly `steps` steps between two synchronisations
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / steps

    # per-call durations of encode and decode on the codec stream: HIP events
    # around each direction's back-to-back layer calls, divided by the layer count;
    # the median over repeated steps (a host stall that lets the queue run dry
    # lands in one repetition only)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    enc_ms, dec_ms = [], []
    for _ in range(max(5, min(steps, 11))):
        hold_queue(torch)
        step(events)
        torch.cuda.synchronize()
        enc_ms.append(events[0].elapsed_time(events[1]) / layers)
        dec_ms.append(events[1].elapsed_time(events[2]) / layers)
    verify(torch, w)
    enc_call = statistics.median(enc_ms)
    dec_call = statistics.median(dec_ms)

    send = w["send"]
    raw_layer = send.total_raw_bytes
    escapes, overflowed = escape_counts(torch, w)
    final = sum(final_payload_bytes(w, layer) for layer in range(layers)) / layers
    cap_bytes = sum(5 * codec_format.top16_escape_capacity(n) for n in send.count_words)
    top16_used = send.total_encoded_bytes - cap_bytes + 5 * escapes / layers
    # algorithmic HBM bytes per call (unused escape slots not counted):
    # encode reads the raw KV and writes the Top-16 payloads (plus, on a layer
    # that overflows, the tiles' presence masks, and for overflowed payloads the
    # masks' read, the fixed6 encode read and its payload write);
    # decode reads the final payloads and writes the raw KV
    fallback_raw = sum(send.raw_bytes[r] for plan in w["plan"] for r in plan["over"]) / layers
    fallback_out = sum(sum(plan.get("sizes", [])) for plan in w["plan"]) / layers
    masks = sum(send.presence_bytes() + 32 * sum(2 * -(-(send.count_words[r] // 2) // 4096)
                                                for r in plan["over"])
                for plan in w["plan"] if plan["over"]) / layers
    b_enc = raw_layer + top16_used + fallback_raw + fallback_out + masks
    if overflowed:
        kept_frac = 1 - overflowed / (layers * send.payload_count)
        b_dec = raw_layer + kept_frac * top16_used + fallback_out
    else:
        b_dec = raw_layer + top16_used
    enc_hbm = b_enc / (enc_call * 1e-3) / 1e9
    dec_hbm = b_dec / (dec_call * 1e-3) / 1e9
    raw_step = raw_layer * layers
    value = raw_step / (ms_per_step * 1e-3) / 1e9
    dominant = (("encode", enc_call, enc_hbm, b_enc) if enc_call >= dec_call
                else ("decode", dec_call, dec_hbm, b_dec))
    kernels = {"encode": "top16_encode_tile+top16_encode_finalize",
               "decode": "top16_decode_tile_dir (escape directory)"}
    if overflowed:
        kernels = {"encode": "top16 probe encode (presence masks; palettes in its finalize "
                             "launch) + palette_encode_tile (fixed6)",
                   "decode": "palette_decode_tile (fixed6)"}

    traffic, traffic_source = measured_traffic(name, dominant[0], bool(overflowed))
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s raw bf16 through encode+decode",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u16 (bf16 bit patterns, integer codec)",
        "data": (f"synthetic seeded (seed {args.seed}); K=N(0,1)*logU[0.1,10] per channel, "
                 f"V=N(0,0.5)" + (f", {w['outliers']:.0%} outliers +-logU[1e2,1e4]"
                                  if w["outliers"] else "")),
        "config": {
            "workload": name,
            "layers": layers,
            "kv_heads": w["shape"].kv_heads,
            "head_dim": w["shape"].head_dim,
            "block_size": w["shape"].block_size,
            "requests": len(w["blocks"]),
            "tokens": [b * w["shape"].block_size for b in w["blocks"]][:8],
            "pool_blocks": w["pool"],
            "raw_bytes_per_step": raw_step,
        },
        "encode": {
            "raw_GBps": round(raw_layer / (enc_call * 1e-3) / 1e9, 2),
            "hbm_GBps": round(enc_hbm, 2),
            "hbm_frac": round(enc_hbm / HBM_PEAK_GBPS, 4),
            "ms_per_layer_call": round(enc_call, 5),
        },
        "decode": {
            "raw_GBps": round(raw_layer / (dec_call * 1e-3) / 1e9, 2),
            "hbm_GBps": round(dec_hbm, 2),
            "hbm_frac": round(dec_hbm / HBM_PEAK_GBPS, 4),
            "ms_per_layer_call": round(dec_call, 5),
        },
        "compression_ratio": round(raw_layer / final, 5),
        "escapes_per_layer": round(escapes / layers, 1),
        "overflowed_payloads": overflowed,
        "roofline": {
            "kernel": kernels[dominant[0]],
            "bound": "hbm",
            "achieved": round(dominant[2], 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dominant[2] / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "algorithmic_bytes_per_call": int(dominant[3]),
            "ms_per_call": round(dominant[1], 5),
        },
        "wall_s_timed": round(wall, 3),
        "verified": True,
    }
    if headline:
        result["graph_replay"] = time_graph_replay(torch, step, w, steps,
                                                   raw_bytes=raw_layer * layers)
        result["exponent_histogram"] = time_histogram(torch, sz, w)
        result["codec_writeback"] = time_writeback(torch, sz, w)
        result["torchop_sender"] = time_torchop_sender(torch, sz, w)
        result["dropin_per_request"] = time_dropin(torch, sz, w)
        result["staging_overlap"] = time_overlap(torch, sz, w)
        result["connector_layer"] = time_connector(torch, sz, w)
        if not args.no_cpu_baseline:
            base = cpu_baseline(torch, w, args.cpu_baseline_layers, args.cpu_baseline_seconds)
            base["legs"] = {"ref-cpu-c": {k: base[k] for k in ("value", "cores", "sample")},
                            "ref-cpu-torch": cpu_baseline_torch(torch, w,
                                                                args.cpu_baseline_seconds),
                            "python_decoder": python_decoder_rate(w)}
            result["cpu_baseline"] = base
    elif name in SUB_CPU_BASELINE and not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, w, 1, SUB_CPU_SECONDS)
    if not headline and name == "llama32-1b-contiguous":
        # launch-bound layers: the same step replayed from a HIP graph, per layer too
        replay = time_graph_replay(torch, step, w, steps, raw_bytes=raw_layer * layers)
        if "ms_per_step" in replay:
            replay["us_per_layer_encode_plus_decode"] = round(replay["ms_per_step"] * 1e3 / layers,
                                                              2)
        result["graph_replay"] = replay
    if w["plan"][0]["over"]:
        result["dropin_fixed6_per_request"] = time_dropin_fixed6(torch, sz, w)
        if not headline:
            # the connector's overflow path: Top-16 attempt, fixed6 fallback, backoff
            result["connector_layer"] = time_connector(torch, sz, w)
    return result




def _sub_summary(result: dict) -> dict:
    """The fields of a non-headline configuration carried in the headline line."""
    keep = ("metric", "value", "unit", "ms_per_step", "steps", "config", "encode", "decode",
            "compression_ratio", "escapes_per_layer", "overflowed_payloads", "roofline",
            "verified", "ms_per_layer_call", "escape_fraction",
            "max_rel_error_vs_decode_then_attend", "decode_only_ms_per_layer", "mfma_TFLOPs",
            "dtype", "data", "dropin_fixed6_per_request", "connector_layer", "cpu_baseline",
            "graph_replay")
    return {k: result[k] for k in keep if k in result}


def _free(torch) -> None:
    import gc

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def main() -> int:
    args = parse_args()
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary), indent=1))
        return 0
    if args.counter_summary:
        print(json.dumps(counter_summary(args.counter_summary), indent=1))
        return 0
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(per-request and per-layer payloads shard with no exchange)"}))
        return 2
    import torch

    from unchainkv_amd import splitzip_cuda as sz
    from unchainkv_amd import workloads

    if not sz.available():
        raise RuntimeError(f"HIP codec library not loaded: {sz.load_error()}")

    def run(name, headline):
        if name == "llama3-8b-decode-attention":
            return run_attention(args, torch, sz, workloads, headline)
        return run_codec(args, torch, sz, workloads, name, headline)

    result = run(args.workload, True)
    if not args.profile_steps and args.configs == "all":
        # every other configuration of the benchmark, shorter: its per-call rates,
        # roofline fraction, ratio and verification
        _free(torch)
        subs = {}
        for name in WORKLOADS:
            if name == args.workload:
                continue
            t0 = time.perf_counter()
            sub = _sub_summary(run(name, False))
            sub["run_s"] = round(time.perf_counter() - t0, 1)
            subs[CONFIG_OF[name]] = dict(workload=name, **sub)
            _free(torch)
        result["configs"] = subs
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
