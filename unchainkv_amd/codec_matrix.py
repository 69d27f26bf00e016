"""One codec correctness and stage-timing point through the drop-in per-request API.

The reference measures its codec with ``scripts/bench_codec_matrix.py``: one request
of ``--tokens`` tokens of a model's KV geometry, its blocks laid out in ``--runs``
contiguous runs, filled with a per-layer pattern, then per iteration gathered into a
contiguous source (``pack``), encoded (``encode_top16`` / ``encode_bf16`` or the raw
mode-6 copy), copied to pinned host memory (``d2h``) and restored (host-to-device
copy, then ``decode_top16`` / ``decode_fixed6`` or the raw ``index_copy_``) into a
receiver cache through the same block ids. Every layer is checked bit for bit
first; the last layer is then timed with CUDA events per stage. This module is
that harness for this library (same command line, same JSON fields), on
``unchainkv_amd.splitzip_cuda``'s drop-in functions, which keep the reference's
signatures:

    python -m unchainkv_amd.codec_matrix --model-config config.json --tokens 4096 \\
        --mode top16 --runs 1 --output result.json

Behaviour followed (``scripts/bench_codec_matrix.py``): run layout :15-25, run count
:28-31, statistics :33-44, geometry :47-54, fill pattern :104-118, pack :120-124,
encode :126-133, restore :135-158, stage events :160-188, checks :190-221, result
:223-253.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
import statistics
import zlib
from pathlib import Path

STAGES = ("pack_ms", "encode_ms", "d2h_ms", "restore_ms", "total_ms")
MODE_BYTE = {"top16": 5, "fixed6": 3, "raw": 6}


def block_ids_for_runs(blocks: int, requested_runs: int) -> list[int]:
    """``blocks`` block ids in min(blocks, runs) contiguous runs whose lengths differ
    by at most one (the longer ones first), one unused id between runs."""
    if blocks <= 0 or requested_runs <= 0:
        raise ValueError("blocks and runs must be positive")
    runs = min(blocks, requested_runs)
    base, extra = divmod(blocks, runs)
    ids: list[int] = []
    next_id = 0
    for run in range(runs):
        length = base + (1 if run < extra else 0)
        ids += list(range(next_id, next_id + length))
        next_id += length + 1  # leave a gap
    return ids


def count_runs(ids: list[int]) -> int:
    """Maximal runs of consecutive ids in list order."""
    if not ids:
        return 0
    return 1 + sum(1 for a, b in zip(ids, ids[1:]) if b != a + 1)


def summary(values: list[float]) -> dict[str, float]:
    """Mean with its normal 95 % interval, median and nearest-rank 95th percentile."""
    ordered = sorted(values)
    n = len(ordered)
    mean = statistics.fmean(ordered)
    half = 1.96 * statistics.stdev(ordered) / math.sqrt(n) if n > 1 else 0.0
    return {"mean": mean, "mean_ci95_low": mean - half, "mean_ci95_high": mean + half,
            "p50": statistics.median(ordered),
            "p95": ordered[max(0, math.ceil(0.95 * n) - 1)]}


def load_geometry(config_path: Path) -> dict[str, int]:
    """Layers, KV heads and head dim of a Hugging Face model config.json."""
    cfg = json.loads(Path(config_path).read_text(encoding="utf-8"))
    heads = int(cfg["num_attention_heads"])
    return {"layers": int(cfg["num_hidden_layers"]),
            "kv_heads": int(cfg.get("num_key_value_heads", heads)),
            "head_dim": int(cfg.get("head_dim", int(cfg["hidden_size"]) // heads))}


def fill_words(mode: str, layer: int, codebooks: bytes) -> tuple[int, int, int | None]:
    """(K word, V word, escape word or None) of the harness's fill for one layer:
    Top-16 fills each plane with its codebook's first exponent and puts an exponent
    outside the codebook at every 200th word; fixed6 and raw use fixed words."""
    if mode == "top16":
        book = codebooks[32 * layer:32 * layer + 32]
        escape = next(e for e in range(1, 255) if e not in book)
        return book[0] << 7 | 0x15, book[16] << 7 | 0x2A, escape << 7 | 0x33
    if mode == "fixed6":
        return 0x7F15, 0x802A, None
    return 0x3F95, 0xC02A, None


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--model-config", required=True, type=Path)
    p.add_argument("--tokens", required=True, type=int)
    p.add_argument("--mode", required=True, choices=tuple(MODE_BYTE))
    p.add_argument("--runs", required=True, type=int)
    p.add_argument("--block-tokens", type=int, default=16)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--iterations", type=int, default=1000)
    p.add_argument("--device", type=int, default=0)
    p.add_argument("--library", help="path of the codec library (UNCHAIN_KV_SPLITZIP_LIB)")
    p.add_argument("--output", required=True, type=Path)
    args = p.parse_args(argv)
    if args.tokens <= 0 or args.tokens % args.block_tokens:
        raise ValueError("tokens must be a positive multiple of block-tokens")
    return args


class _Point:
    """Buffers and stages of one harness point."""

    def __init__(self, args, geometry, torch, sz) -> None:
        self.args, self.torch, self.sz = args, torch, sz
        self.device = torch.device("cuda", args.device)
        self.blocks = args.tokens // args.block_tokens
        self.block_words = args.block_tokens * geometry["kv_heads"] * geometry["head_dim"]
        self.block_ids = block_ids_for_runs(self.blocks, args.runs)
        self.runs = count_runs(self.block_ids)
        dev = self.device
        self.ids = torch.tensor(self.block_ids, dtype=torch.int64, device=dev)
        shape = (2, self.blocks, self.block_words)
        self.source = torch.empty(shape, dtype=torch.bfloat16, device=dev)
        cache_shape = (2, max(self.block_ids) + 1, self.block_words)
        self.cache = torch.empty(cache_shape, dtype=torch.bfloat16, device=dev)
        self.target = torch.zeros_like(self.cache)
        self.pack = torch.empty_like(self.source)
        self.raw_bytes = self.source.numel() * self.source.element_size()
        # the reference sizes its payload buffers at the raw bytes + 1 (raw mode's
        # mode byte); the drop-in encoders need no more room than that
        self.encoded = torch.empty(self.raw_bytes + 1, dtype=torch.uint8, device=dev)
        self.received = torch.empty_like(self.encoded)
        self.raw_received = torch.empty_like(self.source)
        self.host = torch.empty(self.raw_bytes + 1, dtype=torch.uint8, pin_memory=True)
        self.stream = torch.cuda.current_stream(dev)

    def prepare(self, layer: int) -> None:
        k, v, escape = fill_words(self.args.mode, layer, self.sz._TOP16_CODEBOOKS)
        words = self.source.view(self.torch.int16)
        as_int16 = lambda w: w - 0x10000 if w >= 0x8000 else w  # noqa: E731
        words[0].fill_(as_int16(k))
        words[1].fill_(as_int16(v))
        if escape is not None:
            words.reshape(-1)[::200].fill_(as_int16(escape))
        self.cache.index_copy_(1, self.ids, self.source)

    def packed(self):
        if self.runs == 1:
            first = self.block_ids[0]
            return self.cache[:, first:first + self.blocks]
        self.torch.index_select(self.cache, 1, self.ids, out=self.pack)
        return self.pack

    def encode(self, current, layer: int) -> int:
        mode = self.args.mode
        if mode == "top16":
            return int(self.sz.encode_top16(current, self.encoded, layer) or 0)
        if mode == "fixed6":
            return int(self.sz.encode_bf16(current, self.encoded, bits=6) or 0)
        self.encoded[0].fill_(MODE_BYTE["raw"])
        self.encoded[1:].copy_(current.reshape(-1).view(self.torch.uint8))
        return self.raw_bytes + 1

    def restore(self, size: int, layer: int) -> int:
        mode = self.args.mode
        if mode == "raw":
            self.raw_received.view(self.torch.uint8).reshape(-1).copy_(self.host[1:size],
                                                                      non_blocking=True)
            self.target.index_copy_(1, self.ids, self.raw_received)
            return self.raw_bytes
        self.received[:size].copy_(self.host[:size], non_blocking=True)
        if mode == "top16":
            got = self.sz.decode_top16(self.received[:size], self.target, self.block_ids,
                                       self.raw_bytes, layer)
        else:
            got = self.sz.decode_fixed6(self.received[:size], self.target, self.block_ids,
                                        self.raw_bytes)
        return int(got or 0)

    def run_once(self, layer: int):
        """Stage times (ms, CUDA events on the current stream), payload size, source."""
        torch = self.torch
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(8)]
        ev[0].record(self.stream)
        current = self.packed()
        ev[1].record(self.stream)
        ev[2].record(self.stream)
        size = self.encode(current, layer)
        if size <= 0:
            raise RuntimeError(f"{self.args.mode} encoder failed")
        ev[3].record(self.stream)
        ev[4].record(self.stream)
        self.host[:size].copy_(self.encoded[:size], non_blocking=True)
        ev[5].record(self.stream)
        ev[6].record(self.stream)
        copied = self.restore(size, layer)
        ev[7].record(self.stream)
        ev[7].synchronize()
        if copied != self.raw_bytes:
            raise RuntimeError(f"restore copied {copied}/{self.raw_bytes} bytes")
        times = dict(zip(STAGES, (ev[0].elapsed_time(ev[1]), ev[2].elapsed_time(ev[3]),
                                  ev[4].elapsed_time(ev[5]), ev[6].elapsed_time(ev[7]),
                                  ev[0].elapsed_time(ev[7]))))
        return times, size, current

    def differences(self, current) -> int:
        restored = self.target.index_select(1, self.ids)
        return int(self.torch.count_nonzero(restored.view(self.torch.int16)
                                            != current.view(self.torch.int16)).item())


def measure(args) -> dict:
    """The harness point described by ``args``; raises on any mismatch."""
    if args.library:
        import os

        os.environ["UNCHAIN_KV_SPLITZIP_LIB"] = str(args.library)
    import torch

    from . import splitzip_cuda as sz

    if not sz.available():
        raise RuntimeError(f"HIP codec library not loaded: {sz.load_error()}")
    geometry = load_geometry(args.model_config)
    if args.mode == "top16" and len(sz._TOP16_CODEBOOKS) // 32 < geometry["layers"]:
        raise RuntimeError("Top-16 codebooks do not cover every model layer")
    torch.cuda.set_device(args.device)
    pt = _Point(args, geometry, torch, sz)
    checks = []
    current, size = None, 0
    for layer in (range(geometry["layers"]) if args.mode == "top16" else range(1)):
        pt.prepare(layer)
        _, size, current = pt.run_once(layer)
        diff = pt.differences(current)
        mode_byte = int(pt.host[0].item())
        if diff or mode_byte != MODE_BYTE[args.mode]:
            raise RuntimeError(f"layer {layer} mismatch: differences={diff} mode={mode_byte}")
        checks.append({"layer": layer, "bitwise_differences": diff, "payload_mode": mode_byte})
    last = geometry["layers"] - 1 if args.mode == "top16" else 0
    for _ in range(args.warmup):
        pt.run_once(last)
    samples: dict[str, list[float]] = {name: [] for name in STAGES}
    for _ in range(args.iterations):
        times, size, current = pt.run_once(last)
        for name in STAGES:
            samples[name].append(times[name])
    final_diff = pt.differences(current)
    if final_diff:
        raise RuntimeError(f"timed restore has {final_diff} bitwise differences")
    crc = zlib.crc32(memoryview(pt.host[:size].numpy())) & 0xFFFFFFFF
    config_sha = hashlib.sha256(Path(args.model_config).read_bytes()).hexdigest()
    return {
        "passed": True, "model_config": str(args.model_config),
        "model_config_sha256": config_sha, "gpu": torch.cuda.get_device_name(pt.device),
        "geometry": geometry, "tokens": args.tokens, "block_tokens": args.block_tokens,
        "blocks": pt.blocks, "requested_runs": args.runs, "actual_runs": pt.runs,
        "mode": args.mode, "raw_bytes": pt.raw_bytes, "encoded_bytes": size,
        "encoded_crc32": crc, "warmup": args.warmup, "iterations": args.iterations,
        "layer_checks": checks, "final_bitwise_differences": final_diff,
        "timing_ms": {name: summary(values) for name, values in samples.items()},
        "samples_ms": samples,
    }


def main(argv=None) -> None:
    args = parse_args(argv)
    result = measure(args)
    args.output.parent.mkdir(parents=True, exist_ok=True)
    args.output.write_text(json.dumps(result, indent=2, sort_keys=True) + "\n", encoding="utf-8")


if __name__ == "__main__":
    main()
