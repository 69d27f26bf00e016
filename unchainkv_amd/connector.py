"""The codec half of UnchainKV's vLLM connector, on the MI355X codec.

The reference connector (src/unchain_kv/vllm_connector.py) encodes each request's
KV blocks in its per-layer save hook and restores them in its per-layer load hook.
This module keeps that codec behaviour and its knobs, batched per layer:

* policy: Top-16 for payloads of at least 1 MiB when enabled, with the per-layer
  overflow backoff (windows 1, 2, 4 ... up to the cooldown cap, one probe in
  flight, stale results ignored; :2906-3021); a layer whose Top-16 encode declines
  is marked unavailable and uses fixed6 from then on (:3111-3118); fixed5 where
  enabled, downgraded to fixed6 for a layer after it declines or overflows;
* save (``save_kv_layer``): every request of the layer is encoded by one batched
  launch per codec (gathering the blocks in the kernel), then copied to pinned host
  memory from a reusable pool on a copy stream that waits for the forward stream
  (:3406-3458), so later forward kernels do not wait for the copy; ``release``
  returns a layer's pinned buffers once its payloads are sent;
* codec writeback (``CodecConfig.writeback`` without ``preserve_source``,
  :3460-3563): a Top-16 payload whose request holds one contiguous run of blocks is
  moved into those blocks (K-plane run, then V-plane run) by one launch per layer
  and copied to the host from there, so the codec buffer is released at once;
  requests with fragmented block tables are skipped, as in the reference; in the
  early stage the move is deferred until ``finish_deferred_writebacks`` (:3565-3718);
* ready (``ready``): after the copy, Top-16 (and fixed5) payloads whose byte 0 is
  255 are re-encoded as fixed6, and fixed6 overflow falls back to raw mode 6
  (``[6] + raw bytes``) (:4526-4665);
* load (``load_kv_layer`` / ``load_kv_layer_batch``): the restore validation of
  ``_copy_splitzip_bf16_native_blocks`` (:5098-5313) and GPU decode + scatter of
  modes 0-5 (0, 1 and 2, the reference's torch-op codecs, in one launch), raw copy
  of mode 6.

Everything runs on the HIP library; there is no CPU codec path. A request below
1 MiB is sent in the reference's torch-op formats (modes 2, 0, 1, in the
reference's order of preference) unless Top-16 with native decode is enabled
(``prefer_native``, :3043-3046), and as raw words (``raw_passthrough``) when none
of them is smaller (:2685-2711). The KV blocks of a saved layer must stay unchanged until ``ready``
returns: the fallback re-encodes read them again (the reference keeps a gathered
copy instead). The writeback therefore skips an overflowed payload on the GPU (its
mode byte is checked there), leaving its blocks intact for the fixed6 re-encode;
the blocks of a payload that was written back hold the payload afterwards, which
is why the reference only overwrites when neither prefix caching nor chunked
prefill may reuse them (``preserve_source``).
"""

from __future__ import annotations

import os
import weakref
from dataclasses import dataclass, field

from . import codec_format, frames
from .backoff import Top16Backoff
from .staging import CopyStreams, HostCopier, PinnedPool
from .codebooks import summarize_symbol_counts
from .trace import TraceWriter

TOP16_MIN_BYTES = 1 << 20


def _env_int(env, name: str, default: int) -> int:
    value = env.get(name, "")
    return int(value) if value not in {None, ""} else default


def _env_int_set(env, name: str) -> set[int]:
    value = env.get(name, "")
    return {int(item) for item in value.replace(" ", ",").split(",") if item}


@dataclass
class CodecConfig:
    """Codec knobs of the connector (vllm_connector.py:384-449)."""
    top16: bool = False                   # UNCHAIN_KV_SPLITZIP_TOP16
    fixed5: bool = False                  # UNCHAIN_KV_SPLITZIP_FIXED5
    fixed5_layers: set = field(default_factory=set)  # UNCHAIN_KV_SPLITZIP_FIXED5_LAYERS
    top16_max_cooldown: int = 32          # UNCHAIN_KV_SPLITZIP_TOP16_MAX_COOLDOWN
    native_decode: bool = True            # UNCHAIN_KV_SPLITZIP_NATIVE_DECODE (decode is always GPU)
    writeback: bool = False               # UNCHAIN_KV_CODEC_WRITEBACK (default: on with Top-16)
    # prefix caching or chunked prefill may reuse the sender's blocks: no overwrite
    # (the reference derives this from the vLLM config, vllm_connector.py:442-444)
    preserve_source: bool = False
    # caps of the pinned staging pool (0: none), vllm_connector.py:480-486
    host_mirror_layers: int = 0           # UNCHAIN_KV_HOST_MIRROR_LAYERS (buffers)
    host_mirror_bytes: int = 0            # UNCHAIN_KV_HOST_MIRROR_BYTES
    # 2: fixed6 layers send a contiguous request as two half-payloads in KVC2
    # frames (vllm_connector.py:446-447, 2718-2799); anything else: one payload
    chunks: int = 1                       # UNCHAIN_KV_SPLITZIP_CHUNKS
    # GPU event timing of each layer's encodes and copies in the
    # splitzip_payload_ready trace event (vllm_connector.py:473, 4634-4664)
    trace_cuda: bool = False              # UNCHAIN_KV_TRACE_CUDA
    # requests of fewer blocks bypass the codec: no payload is made for them and the
    # transport sends their blocks as they are (vllm_connector.py:385, 5315-5321)
    min_blocks: int = 0                   # UNCHAIN_KV_CODEC_MIN_BLOCKS

    @classmethod
    def from_env(cls, env=None) -> "CodecConfig":
        env = os.environ if env is None else env
        top16 = _env_int(env, "UNCHAIN_KV_SPLITZIP_TOP16", 0) > 0
        return cls(
            top16=top16,
            fixed5=_env_int(env, "UNCHAIN_KV_SPLITZIP_FIXED5", 0) > 0,
            fixed5_layers=_env_int_set(env, "UNCHAIN_KV_SPLITZIP_FIXED5_LAYERS"),
            top16_max_cooldown=max(1, _env_int(env, "UNCHAIN_KV_SPLITZIP_TOP16_MAX_COOLDOWN", 32)),
            native_decode=_env_int(env, "UNCHAIN_KV_SPLITZIP_NATIVE_DECODE", 1) > 0,
            writeback=_env_int(env, "UNCHAIN_KV_CODEC_WRITEBACK", int(top16)) > 0,
            host_mirror_layers=max(0, _env_int(env, "UNCHAIN_KV_HOST_MIRROR_LAYERS", 0)),
            host_mirror_bytes=max(0, _env_int(env, "UNCHAIN_KV_HOST_MIRROR_BYTES", 0)),
            chunks=2 if _env_int(env, "UNCHAIN_KV_SPLITZIP_CHUNKS", 1) == 2 else 1,
            trace_cuda=_env_int(env, "UNCHAIN_KV_TRACE_CUDA", 0) > 0,
            min_blocks=max(0, _env_int(env, "UNCHAIN_KV_CODEC_MIN_BLOCKS", 0)),
        )


# payload modes of the reference's torch-op codecs, restored by one decode launch
TORCHOP_MODES = (codec_format.MODE_PALETTE, codec_format.MODE_NIBBLES, codec_format.MODE_SIGNMAG)
TORCHOP = "torchop"

# bits of a payload as the reference's _SplitzipCudaPayload records them
BITS_TOP16, BITS_FIXED5, BITS_FIXED6, BITS_RAW = 4, 5, 6, 16
# payloads the reference makes outside _SplitzipCudaPayload, which records no bits:
# the torch-op formats (modes 0, 1, 2) and raw words sent with codec raw_passthrough
BITS_TORCHOP, BITS_PASSTHROUGH = 8, 0


def _contiguous_runs(values) -> tuple[tuple[int, int], ...]:
    """(start, count) runs of consecutive ids, in order (vllm_connector.py:148-161)."""
    runs = []
    for value in values:
        value = int(value)
        if runs and value == runs[-1][0] + runs[-1][1]:
            runs[-1][1] += 1
        else:
            runs.append([value, 1])
    return tuple((start, count) for start, count in runs)
@dataclass
class LayerPayload:
    """One request's payload of a layer (the fields of the reference's
    ``_SplitzipCudaPayload`` that the transport and the policy use)."""
    request: int
    block_ids: list
    raw_bytes: int
    bits: int
    requested_bits: int
    epoch: int = -1
    probe: bool = False
    fallback: bool = False
    encoded_bytes: int = 0
    view: memoryview | None = None
    writeback: bool = False          # moved into its own blocks before the host copy
    writeback_segments: int = 0
    deferred_writeback: bool = False  # early stage: moved by finish_deferred_writebacks
    _group: int = -1
    _offset: int = 0
    _status: int = -1                # index of its mode byte in the group's status copy
    _mask_first: int = -1            # first high-byte presence mask in the layer's masks
    _info_index: int = -1            # its palette record in the layer's probe records
    _overflow: bool = False          # overflowed, found from its mode byte alone (deferred copy)
    chunk_index: int = 0             # which half of the request's blocks (two-chunk frames)
    chunks_in_layer: int = 1
    request_blocks: int = 0          # blocks of the whole request, for a chunk's frame

    @property
    def codec(self) -> str:
        return "raw_passthrough" if self.bits == BITS_PASSTHROUGH else "splitzip_bf16"

    def metadata(self, layer_index: int, block_words: int) -> dict:
        """Receiver metadata of a compressed-native layer payload."""
        return {"block_count": len(self.block_ids), "raw_block_size": 2 * 2 * block_words,
                "raw_bytes": self.raw_bytes, "codec": self.codec,
                "encoded_bytes": self.encoded_bytes, "_layer_index": layer_index}


@dataclass
class PendingLayer:
    layer_index: int
    kv_layer: object
    block_words: int
    payloads: list
    groups: list = field(default_factory=list)  # (host array, event, device buffer, status)
    slots: list = field(default_factory=list)   # (pinned pool buffer, lease) behind the arrays
    started: float = 0.0
    presence: object = None  # high-byte presence masks of the Top-16 group (probe encodes)
    palette_info: object = None  # the probe encode's palette record per Top-16 member
    # Top-16 groups whose payload copy waits for their mode bytes:
    # (members, encode result, host array of the mode bytes, its copy event)
    deferred: list = field(default_factory=list)
    timing: list = field(default_factory=list)  # ("encode" | "d2h", start, end) GPU events
    d2h_bytes: int = 0       # bytes queued for the host so far (the layer's PCIe traffic)
    ready_done: bool = False  # ready() has returned: copies complete, overflows settled


class SplitzipLayerCodec:
    """Per-layer save/load codec hooks of one connector worker."""

    def __init__(self, config: CodecConfig | None = None, *, trace=None, codebooks=None,
                 lib=None) -> None:
        config = CodecConfig.from_env() if config is None else config
        self.config = config
        self.trace = trace if trace is not None else TraceWriter(None)
        self.codebooks = {int(k): bytes(v) for k, v in (codebooks or {}).items()}
        self._sz = lib
        # policy state, under the reference connector's names
        self.splitzip_top16 = config.top16
        self.splitzip_fixed5 = config.fixed5
        self.splitzip_fixed5_layers = set(config.fixed5_layers)
        self.splitzip_top16_max_cooldown_payloads = max(1, int(config.top16_max_cooldown))
        self._splitzip_fixed6_layers: set[int] = set()
        self.top16_gate = Top16Backoff(self.splitzip_top16_max_cooldown_payloads, self.trace.event)
        self._traced_bf16_exponents: set[tuple[str, int]] = set()
        self.codec_writeback = config.writeback and config.top16
        self.codec_writeback_overwrite = self.codec_writeback and not config.preserve_source
        self.pinned = PinnedPool(config.host_mirror_bytes, config.host_mirror_layers)
        self.copy_streams = CopyStreams()
        self.host_copier = HostCopier()
        # batches by block tables: a request keeps its block ids in every layer, so
        # a step's layers share them (built once, ids uploaded once)
        self._batches: dict = {}
        # early-stage Top-16 payloads whose writeback waits for
        # finish_deferred_writebacks: (transfer id, layer) -> (pending layer, payload,
        # encode result, index in the encode group)
        self._deferred_codec_writebacks: dict = {}

    # ------------------------------------------------------------------
    # library

    def _lib(self):
        if self._sz is None:
            from . import splitzip_cuda

            self._sz = splitzip_cuda
        if not self._sz.available():
            raise RuntimeError(f"splitzip HIP library unavailable: {self._sz.load_error()}")
        return self._sz

    def _top16_tables(self, layer_index: int, device):
        import torch

        sz = self._lib()
        if layer_index in self.codebooks:
            return sz.top16_tables_for(self.codebooks[layer_index], device, torch)
        return sz._top16_tables(layer_index, device, torch)

    def _layer_codebooks(self, layer_index: int) -> bytes | None:
        if layer_index in self.codebooks:
            return self.codebooks[layer_index]
        sz = self._lib()
        if 0 <= layer_index < len(sz._TOP16_CODEBOOKS) // 32:
            return sz._TOP16_CODEBOOKS[32 * layer_index:32 * (layer_index + 1)]
        return None

    # ------------------------------------------------------------------
    # exponent statistics (vllm_connector.py:2871-2904)

    def _trace_bf16_exponents(self, kv_layer, block_tables, transfer_id: str,
                              layer_index: int) -> None:
        """Once per (transfer, layer): the ``bf16_exponent_stats`` trace event with
        the K and V exponent histograms of the request's blocks, counted on the GPU
        in place (the reference gathers the blocks and runs torch.bincount per
        plane). Failures become ``bf16_exponent_stats_error`` and allow a retry."""
        key = (transfer_id, layer_index)
        if key in self._traced_bf16_exponents:
            return
        self._traced_bf16_exponents.add(key)
        try:
            sz = self._lib()
            batch = sz.PagedBatch(block_tables, kv_layer[0, 0].numel(), kv_layer.device)
            counts = sz.exponent_histogram_paged(kv_layer, batch)
            if counts is None:
                raise RuntimeError("exponent histogram declined")
            k_counts, v_counts = counts.cpu().tolist()
            self.trace.event("bf16_exponent_stats", transfer=transfer_id, layer=layer_index,
                             k=summarize_symbol_counts(k_counts),
                             v=summarize_symbol_counts(v_counts))
        except Exception as exc:  # noqa: BLE001 - the trace must not break the save path
            self._traced_bf16_exponents.discard(key)
            self.trace.event("bf16_exponent_stats_error", transfer=transfer_id,
                             layer=layer_index, error=str(exc)[:160])

    # ------------------------------------------------------------------
    # Top-16 backoff (behaviour of vllm_connector.py:2906-3021; state machine in
    # backoff.Top16Backoff). The reference's method names are kept as the hooks.

    def _should_try_splitzip_top16(self, layer_index: int, raw_bytes: int):
        if not self.splitzip_top16 or raw_bytes < TOP16_MIN_BYTES:
            return False, -1, False
        return self.top16_gate.admit(layer_index)

    def _finish_splitzip_top16_attempt(self, layer_index: int, epoch: int, probe: bool,
                                       overflow: bool) -> None:
        self.top16_gate.settle(layer_index, epoch, probe, overflow)

    def _disable_splitzip_top16(self, layer_index: int, epoch: int) -> None:
        self.top16_gate.disable(layer_index, epoch)

    def _cancel_splitzip_top16_probe(self, layer_index: int, epoch: int, probe: bool) -> None:
        self.top16_gate.cancel(layer_index, epoch, probe)

    def _two_chunks(self, ids: list) -> bool:
        """A request sent as two half-payloads (_try_send_splitzip_two_chunks,
        vllm_connector.py:2718-2737): chunks = 2 with neither Top-16 nor fixed5
        enabled, and an even number (at least 2) of blocks in one ascending run."""
        return (self.config.chunks == 2 and not self.splitzip_top16 and not self.splitzip_fixed5
                and len(ids) >= 2 and len(ids) % 2 == 0 and len(_contiguous_runs(ids)) == 1)

    def _prefer_native(self, raw_bytes: int) -> bool:
        """The native codec for a payload of 1 MiB or more, or for any payload while
        Top-16 with native decode is enabled; the torch-op formats otherwise
        (vllm_connector.py:3043-3046)."""
        return raw_bytes >= TOP16_MIN_BYTES or (self.splitzip_top16 and self.config.native_decode)

    def _choose_bits(self, layer_index: int, raw_bytes: int):
        """Codec choice of _splitzip_bf16_native_blocks (vllm_connector.py:3078-3094)."""
        top16_requested = self.splitzip_top16 and raw_bytes >= TOP16_MIN_BYTES
        try_top16, epoch, probe = self._should_try_splitzip_top16(layer_index, raw_bytes)
        if try_top16:
            bits = BITS_TOP16
        elif top16_requested:
            bits = BITS_FIXED6
        elif (self.splitzip_fixed5 and layer_index not in self._splitzip_fixed6_layers
              and (not self.splitzip_fixed5_layers or layer_index in self.splitzip_fixed5_layers)):
            bits = BITS_FIXED5
        else:
            bits = BITS_FIXED6
        return bits, epoch, probe

    # ------------------------------------------------------------------
    # save

    @staticmethod
    def _layer_geometry(kv_layer, torch):
        if kv_layer.dim() < 3 or kv_layer.shape[0] != 2 or kv_layer.dtype != torch.bfloat16:
            raise ValueError("a KV layer is a bf16 (2, num_blocks, ...) paged cache")
        return kv_layer[0, 0].numel()

    def _encode_group(self, kind: int, kv_layer, members: list, block_words: int, layer_index: int,
                      pending: PendingLayer | None = None):
        """Batched encode of `members` with codec `kind`; returns (device buffer,
        offsets, sizes, batch) or None when the library declines.

        With `pending`: a Top-16 group that holds a probe (the layer overflowed
        before, so it may again) is encoded as a probe: it also records every
        tile's high-byte presence mask in ``pending.presence`` and every member's
        fixed6/fixed5 palette in ``pending.palette_info``, and leaves an overflowed
        payload's escape slots unplaced (it is re-encoded anyway); a palette group
        whose members all have palettes there is encoded in one pass from them (or
        from their masks, without reading the blocks once more for a presence
        pass)."""
        sz = self._lib()
        batch = self._batch([p.block_ids for p in members], block_words, kv_layer.device)
        if kind == BITS_TOP16:
            tables = self._top16_tables(layer_index, kv_layer.device)
            if tables is None:
                return None
            out = batch.new_payload_buffer()
            presence = info = None
            if pending is not None and any(p.probe for p in members):
                presence = batch.new_presence()
                info = batch.new_palette_info() if presence is not None else None
            got = None
            if presence is not None:
                got = sz.encode_top16_paged(kv_layer, batch, out, batch.workspace(),
                                            tables=tables, presence=presence, palette_info=info)
                if got:
                    pending.presence, pending.palette_info = presence, info
                    for k, (p, first) in enumerate(
                            zip(members, batch.presence_first(range(len(members))))):
                        p._mask_first, p._info_index = first, k
            if not got:
                got = sz.encode_top16_paged(kv_layer, batch, out, batch.workspace(),
                                            tables=tables)
            return (out, batch.out_offsets, batch.encoded_bytes, batch) if got else None
        offsets, sizes, _ = batch.palette_layout(kind)
        out = batch.new_palette_buffer(kind)
        got = None
        if pending is not None and pending.palette_info is not None and \
                all(p._info_index >= 0 for p in members):
            got = sz.encode_bf16_paged(kv_layer, batch, out, None, bits=kind,
                                       palette_info=pending.palette_info,
                                       info_first=[p._info_index for p in members])
        if not got:
            masks = {}
            if pending is not None and pending.presence is not None and \
                    all(p._mask_first >= 0 for p in members):
                masks = {"presence": pending.presence,
                         "presence_first": [p._mask_first for p in members]}
            got = sz.encode_bf16_paged(kv_layer, batch, out, batch.new_palette_workspace(),
                                       bits=kind, **masks)
        return (out, offsets, sizes, batch) if got else None

    BATCH_CACHE = 16

    def _batch(self, tables, block_words: int, device):
        """PagedBatch of these block tables, reused while they recur (the most recent
        BATCH_CACHE table sets are kept)."""
        key = (tuple(tuple(t) for t in tables), block_words, str(device))
        batch = self._batches.pop(key, None)
        if batch is None:
            batch = self._lib().PagedBatch([list(t) for t in tables], block_words, device)
            if len(self._batches) >= self.BATCH_CACHE:
                self._batches.pop(next(iter(self._batches)))
        self._batches[key] = batch  # most recent last
        return batch

    def _host_buffer(self, nbytes: int, torch):
        """(pinned host tensor of nbytes, its pool buffer): from the pool, or a fresh
        pinned tensor (buffer None) when the pool's caps leave none."""
        slot = self.pinned.acquire(nbytes, torch)
        if slot is None:
            self.trace.event("host_mirror_full", bytes=nbytes)
            return torch.empty(nbytes, dtype=torch.uint8, pin_memory=True), None
        return slot.view(nbytes), slot

    def _host_array(self, host, slot):
        """The numpy array over a staging tensor that the payloads' memoryviews are
        taken from. A pool buffer's lease ends at ``release()`` or, for a caller
        that never calls it, once this array and every memoryview of it are gone;
        the pool reuses the buffer only after its last copy has completed."""
        arr = host.numpy()
        if slot is not None:
            weakref.finalize(arr, self.pinned.release, slot, slot.lease)
        return arr

    def _begin_copies(self, device, torch):
        """The copy stream, after it has waited for everything queued so far on the
        current (forward) stream: later forward kernels do not wait for the copies
        (vllm_connector.py:3431-3444)."""
        copy = self.copy_streams.get(device, torch)
        copy.wait_stream(torch.cuda.current_stream(device))
        return copy

    def _gpu_mark(self, stream, torch):
        """A timing event recorded on ``stream`` when GPU timing is traced, else None."""
        if not self.config.trace_cuda:
            return None
        event = torch.cuda.Event(enable_timing=True)
        event.record(stream)
        return event

    def _gpu_span(self, pending: PendingLayer, kind: str, start, stream, torch) -> None:
        if start is not None:
            pending.timing.append((kind, start, self._gpu_mark(stream, torch)))

    def _stage_ranges(self, pending: PendingLayer, device_buffer, ranges, torch):
        """Asynchronous copies of the (offset, length) ranges of a device buffer into
        the same offsets of a pinned host buffer, on the copy stream; returns (host
        array, completion event)."""
        host, slot = self._host_buffer(max(1, device_buffer.numel()), torch)
        arr = self._host_array(host, slot)
        copy = self._begin_copies(device_buffer.device, torch)
        with torch.cuda.stream(copy):
            start = self._gpu_mark(copy, torch)
            for off, length in ranges:
                host[off:off + length].copy_(device_buffer[off:off + length], non_blocking=True)
                pending.d2h_bytes += int(length)
            event = torch.cuda.Event(enable_timing=start is not None)
            event.record(copy)
        if start is not None:
            pending.timing.append(("d2h", start, event))
        # the caching allocator must not hand the buffer out again before the copy
        device_buffer.record_stream(copy)
        self._keep_slot(pending, slot, event)
        return arr, event

    def _stage(self, pending: PendingLayer, device_buffer, torch) -> int:
        """Asynchronous copy of a payload buffer into pinned host memory, on the copy
        stream."""
        arr, event = self._stage_ranges(pending, device_buffer, [(0, device_buffer.numel())], torch)
        pending.groups.append((arr, event, device_buffer, None))
        return len(pending.groups) - 1

    def _stage_now(self, pending: PendingLayer, device_buffer, ranges, torch):
        """_stage_ranges, waited for: the fallback payloads ``ready`` makes."""
        arr, event = self._stage_ranges(pending, device_buffer, ranges, torch)
        event.synchronize()
        return arr

    def _defer_top16(self, pending: PendingLayer, members: list, result, torch) -> None:
        """Queue only the group's mode bytes for the host (one gather launch and a
        small copy); ``ready`` copies the payloads that did not overflow and
        re-encodes the others, so no overflowed Top-16 payload crosses PCIe."""
        out, offsets, _, batch = result
        index = getattr(batch, "_mode_index", None)
        if index is None:
            index = torch.tensor([int(o) for o in offsets], dtype=torch.int64).pin_memory()
            index = batch._mode_index = index.to(out.device, non_blocking=True)
        modes = out.index_select(0, index)
        arr, event = self._stage_ranges(pending, modes, [(0, modes.numel())], torch)
        pending.deferred.append((members, result, arr, event))

    @staticmethod
    def _keep_slot(pending: PendingLayer, slot, event) -> None:
        # the pool reuses the buffer only after release() and the copy's end
        if slot is not None:
            slot.event = event
            pending.slots.append((slot, slot.lease))

    def release(self, pending: PendingLayer) -> None:
        """Returns the layer's pinned buffers to the pool once its payloads have been
        consumed (sent); their memory views must not be used afterwards. Without
        this call the buffers go back once the payloads' memoryviews are gone."""
        for slot, lease in pending.slots:
            self.pinned.release(slot, lease)
        pending.slots.clear()

    def _writeback_members(self, members: list, layer_index: int,
                           payloads: list | None = None, **source) -> list[int]:
        """Indices of the Top-16 members whose blocks are one contiguous run (the
        reference skips fragmented tables, vllm_connector.py:3479-3488) and are not
        blocks of another request of the layer (``payloads``): a block shared with
        another request, as prefix caching shares them, would reach that request's
        fallback re-encode or raw copy holding payload bytes. ``source`` is added to
        the skip events (``source="early"`` for deferred writebacks)."""
        owners: dict[int, int] = {}
        for p in payloads if payloads is not None else members:
            for b in p.block_ids:
                owners[b] = owners.get(b, 0) + 1
        picks = []
        for i, p in enumerate(members):
            runs = _contiguous_runs(p.block_ids)
            if len(runs) != 1:
                self.trace.event("codec_writeback_skip", layer=layer_index, reason="fragmented",
                                 segments=len(runs) * 2, **source)
                continue
            if any(owners[b] > 1 for b in p.block_ids):
                self.trace.event("codec_writeback_skip", layer=layer_index, reason="shared",
                                 **source)
                continue
            if not 0 < p.encoded_bytes < p.raw_bytes:
                continue
            picks.append(i)
        return picks

    def _stage_writeback(self, pending: PendingLayer, members: list, result, torch) -> bool:
        """Codec writeback of the Top-16 group (vllm_connector.py:3460-3563): moves
        the eligible payloads into their own blocks with one launch, then copies every
        payload of the group to pinned host memory, the moved ones from their blocks
        (first the K-plane run, then the V-plane run) and the rest from the codec
        buffer, together with each moved payload's mode byte. Returns False (nothing
        staged) when no payload qualifies or the library declines."""
        out, offsets, sizes, batch = result
        layer = pending.layer_index
        picks = self._writeback_members(members, layer, pending.payloads)
        if not picks:
            return False
        sz = self._lib()
        kv_layer = pending.kv_layer
        if not kv_layer.is_contiguous():
            # a run of blocks is not one contiguous segment (vllm_connector.py:3489-3492)
            for i in picks:
                self.trace.event("codec_writeback_skip", layer=layer, reason="layout")
            return False
        moved, status = sz.writeback_top16_paged(out, batch, kv_layer, picks)
        if not moved:
            for i in picks:
                self.trace.event("codec_writeback_skip", layer=layer, reason="alias")
            return False
        host, slot = self._host_buffer(out.numel(), torch)
        arr = self._host_array(host, slot)
        status_host = torch.empty(len(picks), dtype=torch.uint8, pin_memory=True)
        flat = kv_layer.view(-1).view(torch.uint8)
        plane = 2 * kv_layer.stride(0)
        picked = set(picks)
        copy = self._begin_copies(kv_layer.device, torch)
        with torch.cuda.stream(copy):
            start = self._gpu_mark(copy, torch)
            for i, p in enumerate(members):
                off, size = int(offsets[i]), int(sizes[i])
                if i not in picked:
                    host[off:off + size].copy_(out[off:off + size], non_blocking=True)
                    pending.d2h_bytes += size
                    continue
                start, count = _contiguous_runs(p.block_ids)[0]
                seg = 2 * count * pending.block_words
                k = 2 * start * kv_layer.stride(1)
                head = min(size, seg)
                host[off:off + head].copy_(flat[k:k + head], non_blocking=True)
                pending.d2h_bytes += size
                if size > seg:
                    host[off + seg:off + size].copy_(flat[plane + k:plane + k + size - seg],
                                                     non_blocking=True)
            status_host.copy_(status[:len(picks)], non_blocking=True)
            event = torch.cuda.Event(enable_timing=start is not None)
            event.record(copy)
        if start is not None:
            pending.timing.append(("d2h", start, event))
        out.record_stream(copy)
        status.record_stream(copy)
        self._keep_slot(pending, slot, event)
        # the codec buffer is released now unless an unmoved payload is still read from it
        keep = out if len(picks) < len(members) else None
        pending.groups.append((arr, event, keep, status_host))
        group = len(pending.groups) - 1
        for j, i in enumerate(picks):
            p = members[i]
            p.writeback, p.writeback_segments, p._status = True, 2, j
            self.trace.event("codec_writeback_submitted", layer=layer, bytes=p.encoded_bytes,
                             raw_bytes=p.raw_bytes, segments=2)
        for p, off, size in zip(members, offsets, sizes):
            p._group, p._offset, p.encoded_bytes = group, int(off), int(size)
        return True

    def save_kv_layer(self, layer_index: int, kv_layer, block_tables, *, transfer_ids=None,
                      early: bool = False) -> PendingLayer:
        """Encode every request's blocks of one layer (the save hook's codec step) and
        start the copies to host. ``ready`` returns the payloads. A request with
        fewer than ``CodecConfig.min_blocks`` blocks bypasses the codec and has no
        payload (``LayerPayload.request`` names the request of each payload).

        ``transfer_ids``: one id per block table (default: the request's index),
        which keys the deferred writebacks. ``early``: a save of the early stage,
        while the forward pass may still read the blocks (vllm_connector.py:2148-2165):
        with writeback overwrite, no Top-16 payload is moved into its blocks now; it
        is copied to the host from the codec buffer, and its writeback waits for
        ``finish_deferred_writebacks``, which the save hook calls outside the early
        stage with the step's active transfer ids before it saves
        (vllm_connector.py:2065-2080)."""
        import time

        import torch

        started = time.perf_counter()
        if transfer_ids is None:
            transfer_ids = list(range(len(block_tables)))
        elif len(transfer_ids) != len(block_tables):
            raise ValueError("one transfer id per block table")
        block_words = self._layer_geometry(kv_layer, torch)
        payloads = []
        for r, ids in enumerate(block_tables):
            ids = [int(b) for b in ids]
            if not ids:
                raise ValueError("every request needs at least one block")
            if len(ids) < self.config.min_blocks:
                continue  # _use_compressed_native_codec is false for it
            raw = 2 * len(ids) * block_words * 2
            if self._two_chunks(ids):
                # each half of the blocks is its own payload and frame (fixed6, or a
                # torch-op format below 1 MiB)
                half = len(ids) // 2
                bits = BITS_FIXED6 if self._prefer_native(raw // 2) else BITS_TORCHOP
                for chunk in range(2):
                    part = ids[chunk * half:(chunk + 1) * half]
                    payloads.append(LayerPayload(r, part, raw // 2, bits, bits,
                                                 chunk_index=chunk, chunks_in_layer=2,
                                                 request_blocks=len(ids)))
                continue
            if not self._prefer_native(raw):
                payloads.append(LayerPayload(r, ids, raw, BITS_TORCHOP, BITS_TORCHOP))
                continue
            bits, epoch, probe = self._choose_bits(layer_index, raw)
            payloads.append(LayerPayload(r, ids, raw, bits, bits, epoch, probe))
        pending = PendingLayer(layer_index, kv_layer, block_words, payloads, started=started)
        stream = torch.cuda.current_stream(kv_layer.device)

        if any(p.bits == BITS_TORCHOP for p in payloads):
            mark = self._gpu_mark(stream, torch)
            self._torchop_payloads(pending, torch)
            self._gpu_span(pending, "encode", mark, stream, torch)
            payloads = pending.payloads

        # every group is encoded before the Top-16 writeback overwrites any block
        top_result = None
        top = [p for p in payloads if p.bits == BITS_TOP16]
        if top:
            try:
                mark = self._gpu_mark(stream, torch)
                result = self._encode_group(BITS_TOP16, kv_layer, top, block_words, layer_index,
                                            pending)
                self._gpu_span(pending, "encode", mark, stream, torch)
            except Exception:
                for p in top:
                    self._cancel_splitzip_top16_probe(layer_index, p.epoch, p.probe)
                raise
            if result is None:
                for p in top:
                    self._disable_splitzip_top16(layer_index, p.epoch)
                    p.bits, p.fallback = BITS_FIXED6, True
                self.trace.event("splitzip_top16_fallback", layer=layer_index)
            else:
                for p, size in zip(top, result[2]):
                    p.encoded_bytes = int(size)
                top_result = result
        five = [p for p in payloads if p.bits == BITS_FIXED5]
        if five:
            mark = self._gpu_mark(stream, torch)
            result = self._encode_group(BITS_FIXED5, kv_layer, five, block_words, layer_index)
            self._gpu_span(pending, "encode", mark, stream, torch)
            if result is None:
                self._splitzip_fixed6_layers.add(layer_index)
                for p in five:
                    p.bits, p.fallback = BITS_FIXED6, True
                self.trace.event("splitzip_fixed5_overflow", layer=layer_index)
            else:
                self._assign(pending, five, result, torch)
        six = [p for p in payloads if p.bits == BITS_FIXED6]
        if six:
            mark = self._gpu_mark(stream, torch)
            result = self._encode_group(BITS_FIXED6, kv_layer, six, block_words, layer_index)
            self._gpu_span(pending, "encode", mark, stream, torch)
            if result is None:
                for p in six:
                    p.bits = BITS_RAW
            else:
                self._assign(pending, six, result, torch)
        if top_result is not None:
            if pending.presence is not None:
                # a probe of a layer that overflowed before: its payloads cross PCIe
                # only once their mode bytes show that they fit
                self._defer_top16(pending, top, top_result, torch)
            elif not (self.codec_writeback_overwrite and not early
                      and self._stage_writeback(pending, top, top_result, torch)):
                self._assign(pending, top, top_result, torch)
            if early and self.codec_writeback_overwrite:
                for i, p in enumerate(top):
                    if 0 < p.encoded_bytes < p.raw_bytes:
                        p.deferred_writeback = True
                        self._deferred_codec_writebacks[(transfer_ids[p.request], layer_index)] \
                            = (pending, p, top_result, i)
        self.trace.event("codec_encode_submitted", layer=layer_index, requests=len(payloads),
                         raw_bytes=sum(p.raw_bytes for p in payloads))
        return pending

    # ------------------------------------------------------------------
    # deferred (early-stage) codec writeback (vllm_connector.py:3565-3718)

    def finish_deferred_writebacks(self, layer_index: int, kv_layer, transfer_ids=None) -> int:
        """Moves the deferred Top-16 payloads of ``layer_index`` (of ``transfer_ids``,
        the step's active requests; all of the layer's when None) into their blocks
        of ``kv_layer``, as the reference does at the layer's next save outside the
        early stage (vllm_connector.py:3565-3688): one writeback launch per encode
        group on the current stream, K-plane run first, then the V-plane run. The
        blocks then hold the payloads, so they must not be read as KV again; the
        entries of a request that has finished (its blocks may be reused) are
        dropped with ``cancel_deferred_writebacks`` first. A payload is
        skipped when its layer's ``ready`` has not returned (``d2h_pending``), when
        it overflowed and went to the fallback (``overflow``), when its blocks are
        not one contiguous run (``fragmented``) or are shared with another request
        (``shared``), when the layer is not contiguous (``layout``) or when a run
        overlaps the codec buffer (``alias``). Every entry of the layer and ids is
        dropped, and with it the hold on its codec buffer. Returns the bytes
        moved."""
        if not self._deferred_codec_writebacks:
            return 0
        wanted = None if transfer_ids is None else set(transfer_ids)
        keys = [k for k in self._deferred_codec_writebacks
                if k[1] == layer_index and (wanted is None or k[0] in wanted)]
        groups: dict = {}
        for key in keys:
            pending, p, result, i = self._deferred_codec_writebacks.pop(key)
            p.deferred_writeback = False
            if not pending.ready_done:
                self.trace.event("codec_writeback_skip", layer=layer_index, reason="d2h_pending",
                                 source="early")
            elif p.bits != BITS_TOP16:
                self.trace.event("codec_writeback_skip", layer=layer_index, reason="overflow",
                                 source="early")
            else:
                groups.setdefault(id(result), (pending, result, []))[2].append((i, p))
        moved_total = 0
        for pending, result, entries in groups.values():
            out, _, _, batch = result
            members = [p for _, p in entries]
            picks = self._writeback_members(members, layer_index, pending.payloads,
                                            source="early")
            if not picks:
                continue
            if not kv_layer.is_contiguous():
                for _ in picks:
                    self.trace.event("codec_writeback_skip", layer=layer_index, reason="layout",
                                     source="early")
                continue
            try:
                moved, _ = self._lib().writeback_top16_paged(
                    out, batch, kv_layer, [entries[j][0] for j in picks])
            except Exception as exc:  # the reference traces the error and goes on
                self.trace.event("codec_writeback_error", layer=layer_index,
                                 error=str(exc)[:160], source="early")
                continue
            if not moved:
                for _ in picks:
                    self.trace.event("codec_writeback_skip", layer=layer_index, reason="alias",
                                     source="early")
                continue
            moved_total += moved
            for j in picks:
                p = members[j]
                self.trace.event("codec_writeback_submitted", layer=layer_index,
                                 bytes=p.encoded_bytes, raw_bytes=p.raw_bytes, segments=2,
                                 source="early")
        return moved_total

    def cancel_deferred_writebacks(self, transfer_ids=None, layer_index: int | None = None,
                                   reason: str = "cancelled") -> int:
        """Drops deferred writebacks (of ``transfer_ids`` and ``layer_index`` when
        given) without moving anything, as the reference does when a request
        finishes or its metadata is cleared (vllm_connector.py:3690-3718); returns
        how many were dropped."""
        wanted = None if transfer_ids is None else set(transfer_ids)
        keys = [k for k in self._deferred_codec_writebacks
                if (wanted is None or k[0] in wanted)
                and (layer_index is None or k[1] == layer_index)]
        for key in keys:
            _, p, _, _ = self._deferred_codec_writebacks.pop(key)
            p.deferred_writeback = False
            self.trace.event("codec_writeback_skip", layer=key[1], reason=reason,
                             source="early")
        return len(keys)

    # ------------------------------------------------------------------
    # torch-op formats (vllm_connector.py:3204-3343) and raw passthrough

    def _torchop_group(self, pending: PendingLayer, members: list, torch) -> list:
        """Plans and encodes ``members`` in the torch-op formats (one plan launch, a
        host read of the plans' sizes, one encode launch) and stages the payloads;
        returns the members that no format compresses."""
        sz = self._lib()
        kv_layer = pending.kv_layer
        batch = self._batch([p.block_ids for p in members], pending.block_words, kv_layer.device)
        plans = sz.plan_torchop_paged(kv_layer, batch)
        if plans is None:
            return list(members)
        # the host waits for the plans, as the reference waits for its magnitude
        # range (.item()) and palette (torch.unique) before it sizes a payload
        fields = sz.read_torchop_plans(plans.cpu().numpy())
        sizes = [size for _, size in fields]
        offsets, end = [], 0
        for size in sizes:
            offsets.append(end)
            end += size
        if end:
            out = torch.empty(end, dtype=torch.uint8, device=kv_layer.device)
            if sz.encode_torchop_paged(kv_layer, batch, plans, out, offsets, sizes) != end:
                raise RuntimeError("splitzip torch-op encode declined")
            group = self._stage(pending, out, torch)
            for p, off, size in zip(members, offsets, sizes):
                if size:
                    p._group, p._offset, p.encoded_bytes = group, off, size
        return [p for p, size in zip(members, sizes) if not size]

    def _torchop_payloads(self, pending: PendingLayer, torch) -> None:
        """Encodes the layer's torch-op payloads. A request that no format compresses
        is sent as its raw words (raw_passthrough, vllm_connector.py:2685-2711). A
        two-chunk request whose first half is declined is sent whole instead, with
        the codec choice for its full size (:2741-2747); one whose second half alone
        is declined fails, as the reference's does (:2745-2746)."""
        members = [p for p in pending.payloads if p.bits == BITS_TORCHOP]
        declined = self._torchop_group(pending, members, torch)
        whole = {p.request for p in declined if p.chunks_in_layer == 2 and p.chunk_index == 0}
        if any(p.chunks_in_layer == 2 and p.request not in whole for p in declined):
            raise RuntimeError("splitzip second chunk encode failed")
        passthrough = [p for p in declined if p.chunks_in_layer == 1]
        if whole:
            payloads, again = [], []
            for p in pending.payloads:
                if p.request not in whole or p.chunks_in_layer != 2:
                    payloads.append(p)
                elif p.chunk_index == 0:
                    halves = [q for q in pending.payloads
                              if q.request == p.request and q.chunks_in_layer == 2]
                    ids = [b for q in sorted(halves, key=lambda q: q.chunk_index)
                           for b in q.block_ids]
                    raw = 2 * p.raw_bytes
                    if self._prefer_native(raw):
                        bits, epoch, probe = self._choose_bits(pending.layer_index, raw)
                        payloads.append(LayerPayload(p.request, ids, raw, bits, bits, epoch, probe))
                    else:
                        q = LayerPayload(p.request, ids, raw, BITS_TORCHOP, BITS_TORCHOP)
                        payloads.append(q)
                        again.append(q)
            pending.payloads[:] = payloads
            if again:
                passthrough += self._torchop_group(pending, again, torch)
        if passthrough:
            self._stage_passthrough(pending, passthrough, torch)

    def _gather_raw(self, pending: PendingLayer, members: list, mode_byte: bool, torch):
        """One device buffer of each member's words in block order (the K blocks,
        then the V blocks), starting 256-byte aligned, behind a mode byte 6 when
        ``mode_byte``; returns (buffer, offset of each member's first byte)."""
        kv_layer = pending.kv_layer
        batch = self._batch([p.block_ids for p in members], pending.block_words, kv_layer.device)
        lead = 1 if mode_byte else 0
        layout, end = [], 0
        for p in members:
            at = -(-(end + lead) // 256) * 256 - lead
            layout.append(at)
            end = at + lead + p.raw_bytes
        buf = torch.empty(max(end, 1), dtype=torch.uint8, device=kv_layer.device)
        first = 0
        for p, at in zip(members, layout):
            count = len(p.block_ids)
            if mode_byte:
                buf[at:at + 1].fill_(codec_format.MODE_RAW)
            words = buf[at + lead:at + lead + p.raw_bytes].view(torch.bfloat16)
            torch.index_select(kv_layer, 1, batch.ids[first:first + count],
                               out=words.view((2, count) + tuple(kv_layer.shape[2:])))
            first += count
        return buf, layout

    def _stage_passthrough(self, pending: PendingLayer, members: list, torch) -> None:
        """Raw words sent with codec raw_passthrough (no mode byte), gathered on the
        GPU and staged like the encoded payloads."""
        stream = torch.cuda.current_stream(pending.kv_layer.device)
        mark = self._gpu_mark(stream, torch)
        buf, layout = self._gather_raw(pending, members, False, torch)
        self._gpu_span(pending, "encode", mark, stream, torch)
        group = self._stage(pending, buf, torch)
        for p, at in zip(members, layout):
            p.bits = BITS_PASSTHROUGH
            p._group, p._offset, p.encoded_bytes = group, at, p.raw_bytes

    def _assign(self, pending, members, result, torch) -> None:
        out, offsets, sizes, _ = result
        group = self._stage(pending, out, torch)
        for p, off, size in zip(members, offsets, sizes):
            p._group, p._offset, p.encoded_bytes = group, int(off), int(size)

    # ------------------------------------------------------------------
    # ready: overflow fallback chain (vllm_connector.py:4526-4665)

    def ready(self, pending: PendingLayer) -> list:
        """The layer's payloads once on the host (vllm_connector.py:4526-4665): the
        copies are waited for; Top-16 (and fixed5) payloads that overflowed are
        re-encoded as fixed6 with one launch, and fixed6 overflow falls back to raw
        mode 6. The fallback payloads are staged like the others: pinned pool
        buffers, copies on the copy stream."""
        import time

        import torch

        for host, event, _, _ in pending.groups:
            event.synchronize()
        layer = pending.layer_index
        for p in pending.payloads:
            if p._group >= 0:
                host, _, _, status = pending.groups[p._group]
                if p.writeback:
                    # a payload the GPU did not move (an overflow) left its blocks
                    # intact and the host bytes are not the payload: mark it 255
                    mode = int(status[p._status])
                    overflow = mode != codec_format.MODE_TOP16
                    if overflow:
                        host[p._offset] = codec_format.MODE_OVERFLOW
                    self.trace.event("codec_writeback_done", layer=layer, bytes=p.encoded_bytes,
                                     raw_bytes=p.raw_bytes, segments=p.writeback_segments,
                                     overflow=overflow)
                p.view = memoryview(host)[p._offset:p._offset + p.encoded_bytes]
        for members, result, modes, event in pending.deferred:
            # only the payloads that fit go to the host; the others are re-encoded below
            event.synchronize()
            out, offsets, sizes, _ = result
            fit = [i for i in range(len(members)) if modes[i] == codec_format.MODE_TOP16]
            for i in range(len(members)):
                members[i]._overflow = i not in fit
            if fit:
                ranges = [(int(offsets[i]), int(sizes[i])) for i in fit]
                host = self._stage_now(pending, out, ranges, torch)
                for i, (off, size) in zip(fit, ranges):
                    members[i].view = memoryview(host)[off:off + size]
        pending.deferred.clear()

        def overflowed_payload(p) -> bool:
            return p._overflow or (p.view is not None and p.view[0] == codec_format.MODE_OVERFLOW)

        for p in pending.payloads:
            if p.bits == BITS_TOP16:
                self._finish_splitzip_top16_attempt(layer, p.epoch, p.probe, overflowed_payload(p))
        overflowed = [p for p in pending.payloads
                      if overflowed_payload(p) and p.bits in {BITS_TOP16, BITS_FIXED5}]
        if any(p.bits == BITS_FIXED5 for p in overflowed):
            self._splitzip_fixed6_layers.add(layer)
            self.trace.event("splitzip_fixed5_overflow", layer=layer)
        if overflowed:
            stream = torch.cuda.current_stream(pending.kv_layer.device)
            mark = self._gpu_mark(stream, torch)
            result = self._encode_group(BITS_FIXED6, pending.kv_layer, overflowed,
                                        pending.block_words, layer, pending)
            self._gpu_span(pending, "encode", mark, stream, torch)
            for p in overflowed:
                p.view = None
            if result is not None:
                out, offsets, sizes, _ = result
                host = self._stage_now(pending, out, [(0, out.numel())], torch)
                for p, off, size in zip(overflowed, offsets, sizes):
                    p.view = memoryview(host)[off:off + size]
                    p.encoded_bytes = int(size)
            for p in overflowed:
                p.bits, p.fallback, p._overflow = BITS_FIXED6, True, False
        raws = [p for p in pending.payloads if p.bits != BITS_PASSTHROUGH and (
            p.bits == BITS_RAW or p.view is None or p.view[0] == codec_format.MODE_OVERFLOW)]
        if raws:
            self._stage_raw(pending, raws, torch)
            for _ in raws:
                self.trace.event("splitzip_fixed6_overflow", layer=layer)
        pending.presence = pending.palette_info = None
        fields = {}
        if self.config.trace_cuda:
            # the events have completed: every copy above was waited for
            fields = {
                "bits": [p.bits for p in pending.payloads],
                "fallback": [p.fallback for p in pending.payloads],
                "encode_gpu_s": sum(a.elapsed_time(b) for k, a, b in pending.timing
                                    if k == "encode") / 1000.0,
                "d2h_gpu_s": sum(a.elapsed_time(b) for k, a, b in pending.timing
                                 if k == "d2h") / 1000.0,
                "payload_elapsed_s": time.perf_counter() - pending.started,
            }
        pending.timing.clear()
        pending.ready_done = True
        self.trace.event("splitzip_payload_ready", layer=layer,
                         raw_bytes=sum(p.raw_bytes for p in pending.payloads),
                         encoded_bytes=sum(p.encoded_bytes for p in pending.payloads), **fields)
        return pending.payloads

    def _stage_raw(self, pending: PendingLayer, raws: list, torch) -> None:
        """Raw mode-6 payloads (``[6]`` + the request's words in block order,
        vllm_connector.py:4606-4625): the blocks are gathered on the GPU into one
        buffer behind each payload's mode byte and copied to the host like the
        others."""
        stream = torch.cuda.current_stream(pending.kv_layer.device)
        mark = self._gpu_mark(stream, torch)
        buf, layout = self._gather_raw(pending, raws, True, torch)
        self._gpu_span(pending, "encode", mark, stream, torch)
        host = self._stage_now(pending, buf, [(at, 1 + p.raw_bytes) for p, at in zip(raws, layout)],
                               torch)
        for p, at in zip(raws, layout):
            p.view = memoryview(host)[at:at + 1 + p.raw_bytes]
            p.bits, p.encoded_bytes = BITS_RAW, 1 + p.raw_bytes

    # ------------------------------------------------------------------
    # load: restore validation and dispatch (vllm_connector.py:5098-5313)

    @staticmethod
    def _validate(kv_layer, block_ids, payload, metadata, torch):
        """(mode, raw_bytes, view) for a payload the restore accepts, else None."""
        if kv_layer.dim() < 3 or kv_layer.shape[0] != 2 or not block_ids:
            return None
        if len(set(block_ids)) != len(block_ids) or any(
                b < 0 or b >= kv_layer.shape[1] for b in block_ids):
            return None
        first = kv_layer[:, block_ids[0]]
        raw_bytes = int(metadata.get("raw_bytes", 0))
        n = raw_bytes // 2
        encoded_bytes = int(metadata.get("encoded_bytes", 0))
        expected = len(block_ids) * first.numel() * first.element_size()
        if (kv_layer.dtype != torch.bfloat16 or raw_bytes <= 0 or raw_bytes % 2
                or raw_bytes != expected):
            return None
        view = memoryview(payload).cast("B")
        if encoded_bytes < 1 or len(view) != encoded_bytes:
            return None
        mode = int(view[0])
        if mode not in range(7):
            return None
        if mode == codec_format.MODE_FIXED6 and encoded_bytes != codec_format.fixed6_encoded_size(n):
            return None
        if mode == codec_format.MODE_FIXED5 and encoded_bytes != codec_format.fixed5_encoded_size(n):
            return None
        if mode == codec_format.MODE_TOP16 and encoded_bytes != codec_format.top16_encoded_size(n):
            return None
        if mode == codec_format.MODE_RAW and encoded_bytes != raw_bytes + 1:
            return None
        if mode in TORCHOP_MODES and codec_format.torchop_encoded_size(view, n) != encoded_bytes:
            return None
        return mode, raw_bytes, view

    # ------------------------------------------------------------------
    # wire frames (tcp_data.py:612-652 send, :282-361 receive)

    @staticmethod
    def frames(layer_index: int, payloads, block_words: int, transfer_id: str,
               request_ids) -> list:
        """Compressed-native frames carrying the ready payloads of a layer (parts
        as ``frames.pack_compressed_native`` returns them): KVC1, one per request,
        or KVC2 for each half of a request sent in two chunks;
        ``request_ids[p.request]`` names each request."""
        out = []
        for p in payloads:
            if p.view is None:
                raise ValueError("payload is not ready")
            meta = p.metadata(layer_index, block_words)
            if p.chunks_in_layer > 1:
                # a KVC2 chunk carries the whole request's block count and raw
                # bytes (vllm_connector.py:5551-5563)
                out.append(frames.pack_compressed_native(
                    transfer_id, request_ids[p.request], layer_index, p.view,
                    raw_block_size=meta["raw_block_size"], block_count=p.request_blocks,
                    raw_bytes=meta["raw_block_size"] * p.request_blocks, codec=meta["codec"],
                    chunk_index=p.chunk_index, chunks_in_layer=p.chunks_in_layer))
                continue
            out.append(frames.pack_compressed_native(
                transfer_id, request_ids[p.request], layer_index, p.view,
                raw_block_size=meta["raw_block_size"], block_count=meta["block_count"],
                raw_bytes=meta["raw_bytes"], codec=meta["codec"]))
        return out

    def restore_frames(self, kv_layer, bodies, block_tables: dict) -> dict:
        """Restore received compressed-native frame bodies of one layer into the
        blocks ``block_tables[request_id]``: KVC1 frames whole, KVC2 chunks
        (chunks_in_layer 2) into their half of the block list with raw_bytes
        raw_block_size * blocks (vllm_connector.py:4785-4810), raw_passthrough
        payloads as raw words. Returns {request_id: (blocks, bytes)}; every frame of
        a call must carry the same layer."""
        parsed = [frames.parse_compressed_native(b) for b in bodies]
        if not parsed:
            return {}
        layer = parsed[0].layer_index
        if any(f.layer_index != layer for f in parsed):
            raise ValueError("frames of different layers")
        requests, keys = [], []
        for f in parsed:
            ids = [int(b) for b in block_tables[f.request_id]]
            meta = f.metadata()
            payload = f.payload
            if f.chunks_in_layer > 1:
                if f.chunks_in_layer != 2 or len(ids) % 2:
                    continue
                half = len(ids) // 2
                ids = ids[f.chunk_index * half:(f.chunk_index + 1) * half]
                meta = dict(meta, raw_bytes=f.raw_block_size * len(ids),
                            encoded_bytes=f.encoded_bytes)
            requests.append((ids, payload, meta))
            keys.append(f.request_id)
        results = self.load_kv_layer_batch(layer, kv_layer, requests)
        out: dict = {}
        for key, (blocks, nbytes) in zip(keys, results):
            prev = out.get(key, (0, 0))
            out[key] = (prev[0] + blocks, prev[1] + nbytes)
        return out

    def load_kv_layer(self, kv_layer, block_ids, payloads, metadata) -> tuple[int, int]:
        """Restore one request's layer payload into its blocks; (blocks, bytes) or
        (0, 0) when the payload is refused."""
        if len(payloads) != 1:
            return 0, 0
        return self.load_kv_layer_batch(int(metadata.get("_layer_index", -1)), kv_layer,
                                        [(block_ids, payloads[0], metadata)])[0]

    def load_kv_layer_batch(self, layer_index: int, kv_layer, requests) -> list:
        """Restore every request of a layer: ``requests`` holds (block_ids, payload
        bytes, metadata). Payloads are staged in one pinned buffer, which goes to the
        GPU range by range while the host threads are still staging later payloads,
        and decoded with one launch per payload mode. Returns (blocks, bytes) per
        request."""
        import torch

        sz = self._lib()
        results = [(0, 0)] * len(requests)
        groups: dict[int, list] = {}
        for k, (block_ids, payload, metadata) in enumerate(requests):
            block_ids = [int(b) for b in block_ids]
            if metadata.get("codec") == "raw_passthrough":
                # the native words themselves: restored as a mode-6 payload
                payload = bytes([codec_format.MODE_RAW]) + bytes(payload)
                metadata = dict(metadata, encoded_bytes=len(payload))
            checked = self._validate(kv_layer, block_ids, payload, metadata, torch)
            if checked is None:
                continue
            mode, raw_bytes, view = checked
            # modes 0, 1 and 2 (the torch-op codecs) share one decode launch
            key = TORCHOP if mode in TORCHOP_MODES else mode
            groups.setdefault(key, []).append((k, block_ids, raw_bytes, view))
        if not groups:
            return results
        block_words = kv_layer[0, 0].numel()
        # one pinned staging buffer, each payload's sections starting on a
        # 256-byte boundary (the decode kernels take any offset; whole cache
        # lines per tile span are cheaper)
        header = {codec_format.MODE_TOP16: 5, codec_format.MODE_FIXED6: 65,
                  codec_format.MODE_FIXED5: 33, codec_format.MODE_RAW: 1, TORCHOP: 0}
        layout, end = [], 0
        for mode, members in groups.items():
            for member in members:
                start = -(-(end + header[mode]) // 256) * 256 - header[mode]
                layout.append((mode, member, start))
                end = start + len(member[3])
        batches = {mode: self._batch([m[1] for m in members], block_words, kv_layer.device)
                   for mode, members in groups.items()}
        # the Top-16 payloads' escape directory rides along in the same copy, so
        # their decode is one kernel
        top = groups.get(codec_format.MODE_TOP16)
        dir_at = dir_bytes = 0
        if top:
            dir_bytes = batches[codec_format.MODE_TOP16].directory_bytes()
            if dir_bytes:
                dir_at = -(-end // 256) * 256
                end = dir_at + dir_bytes
        host, slot = self._host_buffer(max(end, 1), torch)
        try:
            host_np = host.numpy()
            device = torch.empty(max(end, 1), dtype=torch.uint8, device=kv_layer.device)

            def upload(lo: int, hi: int) -> None:
                device[lo:hi].copy_(host[lo:hi], non_blocking=True)

            # each range of the staging buffer goes to the GPU as soon as its payload
            # bytes are in place, while the host threads copy the next ones
            payload_end = max((start + len(member[3]) for _, member, start in layout), default=0)
            self.host_copier.copy_streamed(host_np,
                                           [(start, member[3]) for _, member, start in layout],
                                           upload, end=payload_end)
            if dir_bytes:
                tops = [start for m, _, start in layout if m == codec_format.MODE_TOP16]
                # the builder sorts each escape list in place (a reference sender's is in
                # atomic order): a list it reordered goes to the GPU again
                lists = []
                for start, member in zip(tops, top):
                    n = member[2] // 2
                    lo = start + codec_format.top16_sections(n)["escapes"][0]
                    count = min(int.from_bytes(bytes(host_np[start + 1:start + 5]), "little"),
                                codec_format.top16_escape_capacity(n))
                    lists.append((lo, lo + 5 * count, host_np[lo:lo + 5 * count].copy()))
                built = sz.build_directory(host_np, tops, [len(m[3]) for m in top],
                                           batches[codec_format.MODE_TOP16])
                if built is None:
                    dir_bytes = 0
                else:
                    host_np[dir_at:dir_at + dir_bytes] = built
                    upload(dir_at, dir_at + dir_bytes)
                for lo, hi, before in lists:
                    if (before != host_np[lo:hi]).any():
                        upload(lo, hi)
        finally:
            if slot is not None:
                # back to the pool at once (also when staging raised): reused after
                # the host-to-device copies queued so far end
                slot.event = torch.cuda.Event()
                slot.event.record(torch.cuda.current_stream(kv_layer.device))
                self.pinned.release(slot)
        for mode, members in groups.items():
            starts = [start for m, _, start in layout if m == mode]
            batch = batches[mode]
            sizes = [len(m[3]) for m in members]
            if mode == codec_format.MODE_TOP16:
                books = self._layer_codebooks(layer_index)
                if books is None:
                    continue
                directory = device[dir_at:dir_at + dir_bytes] if dir_bytes else None
                copied = sz.decode_top16_paged(device, starts, sizes, kv_layer, batch,
                                               codebooks=books, directory=directory)
                if not copied and directory is not None:
                    # a layout the one-kernel decode does not take: two kernels
                    copied = sz.decode_top16_paged(device, starts, sizes, kv_layer, batch,
                                                   codebooks=books)
            elif mode == TORCHOP:
                copied = sz.decode_torchop_paged(device, starts, sizes, kv_layer, batch)
            elif mode == codec_format.MODE_RAW:
                copied = 0
                for (k, ids, raw_bytes, _), start in zip(members, starts):
                    words = device[start + 1:start + 1 + raw_bytes].view(torch.bfloat16)
                    source = words.reshape((2, len(ids)) + tuple(kv_layer.shape[2:]))
                    index = torch.as_tensor(ids, dtype=torch.long, device=kv_layer.device)
                    kv_layer.index_copy_(1, index, source)
                    copied += raw_bytes
            else:
                bits = 6 if mode == codec_format.MODE_FIXED6 else 5
                copied = sz.decode_bf16_paged(device, starts, sizes, kv_layer, batch, bits=bits)
            if copied:
                for k, ids, raw_bytes, _ in members:
                    results[k] = (len(ids), raw_bytes)
                modes = sorted({int(m[3][0]) for m in members}) if mode == TORCHOP else [mode]
                for m in modes:
                    self.trace.event("splitzip_native_decode",
                                     blocks=sum(len(x[1]) for x in members if int(x[3][0]) == m),
                                     bytes=sum(x[2] for x in members if int(x[3][0]) == m),
                                     mode=m)
        return results
