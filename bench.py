#!/usr/bin/env python3
"""Throughput of the MI355X splitzip Top-16 KV codec (one GPU).

Workload (default ``llama3-8b-paged``): Llama-3-8B-shaped paged KV, 32 layers x
(2, 4096 blocks, 16 tokens, 8 KV heads, 128) bf16, seeded synthetic values
(K = N(0,1) x per-channel scale log-uniform in [0.1, 10], V = N(0, 0.5)); a batch
of 8 requests x 4096 tokens whose block tables are disjoint random slices of one
seeded permutation of the pool; per-layer K/V Top-16 codebooks fit on the same
tensor. One step = for every layer, gather + encode all 8 requests into packed
payloads (one batched launch per layer), then decode + scatter every payload into
a receiver cache through an independent random block table.

The JSON line reports raw bf16 bytes through the round trip per second as
``value``, the encode and decode rates separately, the HBM roofline fraction of
the dominant kernel call from HIP events on the codec's stream, the compression
ratio, and the oracle's multi-threaded CPU codec timed on a bounded sample on
this host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBPS = 8000.0
CALIBRATION_BYTES = 256 << 20
METRIC = "codec encode/decode GB/s of raw bf16 KV (% HBM peak) + compression ratio"


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=30)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", default="llama3-8b-paged",
                   choices=["llama3-8b-paged", "llama32-1b-contiguous", "llama3-70b-tp8-mixed"])
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--cpu-baseline-layers", type=int, default=2,
                   help="layers of the workload the CPU baseline encodes and decodes")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--profile-steps", type=int, default=0,
                   help="only run this many untimed steps (for rocprofv3), then exit")
    return p.parse_args()


def build_workload(torch, sz, workloads, name: str, seed: int):
    """Layers, batches, codebook tables and buffers of one workload."""
    if name == "llama3-8b-paged":
        shape, pool = workloads.LLAMA3_8B, 4096
        blocks = [4096 // shape.block_size] * 8
        layers = shape.layers
    elif name == "llama32-1b-contiguous":
        shape, pool = workloads.LLAMA32_1B, 64
        blocks = [1024 // shape.block_size]
        layers = shape.layers
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
    kv, tables, books, payloads = [], [], [], []
    for layer in range(layers):
        cache = workloads.make_kv_layer(torch, shape, pool, seed=seed, layer=layer, device=device)
        book = workloads.fit_codebook(torch, cache, send_tables)
        kv.append(cache)
        books.append(book)
        tables.append(sz.top16_tables_for(book, device, torch))
        payloads.append(send.new_payload_buffer())
    receiver = [torch.zeros_like(kv[0]) for _ in range(layers)]
    workspace = send.new_workspace()
    return {
        "shape": shape, "pool": pool, "blocks": blocks, "layers": layers, "send": send,
        "recv": recv, "kv": kv, "tables": tables, "books": books, "payloads": payloads,
        "receiver": receiver, "workspace": workspace, "device": device,
    }


def encode_layer(sz, w, layer):
    got = sz.encode_top16_paged(w["kv"][layer], w["send"], w["payloads"][layer], w["workspace"],
                                tables=w["tables"][layer])
    if got != w["send"].total_encoded_bytes:
        raise RuntimeError(f"layer {layer}: paged encode declined ({got})")


def decode_layer(sz, w, layer):
    send = w["send"]
    got = sz.decode_top16_paged(w["payloads"][layer], send.out_offsets, send.encoded_bytes,
                                w["receiver"][layer], w["recv"], tables=w["tables"][layer])
    if got != send.total_raw_bytes:
        raise RuntimeError(f"layer {layer}: paged decode declined ({got})")


def escape_counts(torch, w):
    """Escape entries per layer (from the payload headers) and overflowed payloads."""
    send = w["send"]
    total, overflow = 0, 0
    for layer in range(w["layers"]):
        host = w["payloads"][layer].cpu()
        for off in send.out_offsets:
            head = bytes(host[off:off + 5].tolist())
            total += int.from_bytes(head[1:5], "little")
            overflow += head[0] == 255
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


def cpu_baseline(torch, w, layers: int):
    """The oracle's multi-threaded C codec (gather + canonical encode, then
    decode + scatter) on this host's cores over the first `layers` layers."""
    import numpy as np

    import oracle

    threads = oracle.default_threads()
    shape, pool, send, recv = w["shape"], w["pool"], w["send"], w["recv"]
    bw = shape.block_words
    raw = 0
    t_enc = t_dec = 0.0
    for layer in range(min(layers, w["layers"])):
        kv = w["kv"][layer].view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)
        tab = oracle.top16_tables(w["books"][layer])
        t0 = time.perf_counter()
        out = oracle.encode_paged_batch(kv, pool * bw, bw, bw, send.block_tables, send.out_offsets,
                                        send.out_bytes, tab, threads=threads)
        t1 = time.perf_counter()
        target = np.zeros(kv.size, np.uint16)
        oracle.decode_paged_batch(out, send.out_offsets, target, pool * bw, bw, bw,
                                  recv.block_tables, tab, threads=threads)
        t2 = time.perf_counter()
        t_enc += t1 - t0
        t_dec += t2 - t1
        raw += send.total_raw_bytes
        gpu = w["payloads"][layer].cpu().numpy()
        for off, size in zip(send.out_offsets, send.encoded_bytes):
            if bytes(gpu[off:off + size]) != bytes(out[off:off + size]):
                raise RuntimeError(f"layer {layer}: GPU payload differs from the oracle")
    sample = (f"{min(layers, w['layers'])} of {w['layers']} layers "
              f"({raw / 2**30:.2f} GiB raw bf16) encoded then decoded")
    return {
        "value": round(2 * raw / (t_enc + t_dec) / 1e9, 3),
        "unit": "GB/s raw bf16 (encode+decode round trip)",
        "cores": threads,
        "kind": "port",
        "sample": sample,
        "encode_GBps": round(raw / t_enc / 1e9, 3),
        "decode_GBps": round(raw / t_dec / 1e9, 3),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(per-request/per-layer payloads shard with no exchange, see DESIGN.md)"}))
        return 2
    import torch

    from unchainkv_amd import codec_format
    from unchainkv_amd import splitzip_cuda as sz
    from unchainkv_amd import workloads

    if not sz.available():
        raise RuntimeError(f"HIP codec library not loaded: {sz.load_error()}")
    w = build_workload(torch, sz, workloads, args.workload, args.seed)
    layers = w["layers"]
    stream = torch.cuda.current_stream(w["device"])

    def step(enc_events=None, dec_events=None):
        for layer in range(layers):
            if enc_events:
                enc_events[layer][0].record(stream)
            encode_layer(sz, w, layer)
            if enc_events:
                enc_events[layer][1].record(stream)
        for layer in range(layers):
            if dec_events:
                dec_events[layer][0].record(stream)
            decode_layer(sz, w, layer)
            if dec_events:
                dec_events[layer][1].record(stream)

    if args.profile_steps:
        for _ in range(args.profile_steps):
            step()
        torch.cuda.synchronize()
        verify(torch, w)
        # calibration for HBM counters: one plain copy of a known size (256 MiB
        # read + 256 MiB written) in the same process
        src = torch.empty(CALIBRATION_BYTES // 2, dtype=torch.int16, device=w["device"])
        src.fill_(3)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": args.profile_steps, "workload": args.workload,
                          "calibration_copy_bytes": CALIBRATION_BYTES}))
        return 0

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    verify(torch, w)

    # timed region: exactly `steps` steps between two synchronisations
    t0 = time.perf_counter()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = start.elapsed_time(end)
    ms_per_step = ms_total / args.steps

    # per-call durations of encode and decode on the codec stream
    enc_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(layers)]
    dec_ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(layers)]
    enc_ms, dec_ms = [], []
    for _ in range(max(3, min(args.steps, 10))):
        step(enc_ev, dec_ev)
        torch.cuda.synchronize()
        enc_ms += [a.elapsed_time(b) for a, b in enc_ev]
        dec_ms += [a.elapsed_time(b) for a, b in dec_ev]
    verify(torch, w)
    enc_call = sum(enc_ms) / len(enc_ms)
    dec_call = sum(dec_ms) / len(dec_ms)

    send = w["send"]
    raw_layer = send.total_raw_bytes
    enc_layer = send.total_encoded_bytes
    escapes, overflowed = escape_counts(torch, w)
    esc_layer = escapes / layers
    cap_bytes = sum(5 * codec_format.top16_escape_capacity(n) for n in send.count_words)
    # algorithmic HBM bytes per call: read raw once + write payload once (encode) and
    # the reverse (decode); unused escape slots are not counted
    payload_used = enc_layer - cap_bytes + 5 * esc_layer
    b_call = raw_layer + payload_used
    enc_hbm = b_call / (enc_call * 1e-3) / 1e9
    dec_hbm = b_call / (dec_call * 1e-3) / 1e9
    raw_step = raw_layer * layers
    value = raw_step / (ms_per_step * 1e-3) / 1e9
    dominant = ("encode", enc_call, enc_hbm) if enc_call >= dec_call else ("decode", dec_call, dec_hbm)

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s raw bf16 through encode+decode",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u16 (bf16 bit patterns, integer codec)",
        "data": f"synthetic seeded (seed {args.seed}); K=N(0,1)*logU[0.1,10] per channel, V=N(0,0.5)",
        "config": {
            "workload": args.workload,
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
        "compression_ratio": round(raw_layer / enc_layer, 5),
        "escapes_per_layer": round(esc_layer, 1),
        "overflowed_payloads": overflowed,
        "roofline": {
            "kernel": ("top16_encode_kernel+top16_encode_finalize" if dominant[0] == "encode"
                       else "top16_decode_kernel+top16_patch_escapes"),
            "bound": "hbm",
            "achieved": round(dominant[2], 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(dominant[2] / HBM_PEAK_GBPS, 4),
            "traffic": None,
            "algorithmic_bytes_per_call": int(b_call),
            "ms_per_call": round(dominant[1], 5),
        },
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(torch, w, args.cpu_baseline_layers)
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())
