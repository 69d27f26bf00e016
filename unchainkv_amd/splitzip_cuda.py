"""Drop-in host module for the splitzip bf16 KV codec on MI355X.

Mirrors ``unchain_kv.splitzip_cuda`` (src/unchain_kv/splitzip_cuda.py): the same
function names, argument meanings and return conventions, over the HIP library
``libunchain_kv_splitzip_cuda.so`` built from ``unchainkv_amd/csrc``:

* ``encode_top16`` / ``decode_top16`` / ``encode_bf16`` / ``decode_fixed6``
  return the byte count, ``None`` when the codec declines (library missing,
  wrong device/dtype/layout, precondition failed), and raise ``RuntimeError``
  with ``kvq_splitzip_last_error()`` when a launch fails;
* ``_top16_tables(layer, device, torch)`` builds (and caches per device and
  layer) the 544-byte device table from ``_TOP16_CODEBOOKS``.

Additions (keyword-only or new names, so reference callers are unaffected):

* ``codebooks=`` on ``encode_top16`` / ``decode_top16``: a 32-byte per-layer
  codebook (16 K exponents, then 16 V exponents) instead of the embedded one;
* ``PagedBatch`` + ``encode_top16_paged`` / ``decode_top16_paged``: every
  request of one paged layer in one launch, gathering straight from the block
  table (no packed copy of the request's blocks first).

Everything runs asynchronously on ``torch.cuda.current_stream(device)``.
"""

from __future__ import annotations

import array
import ctypes
import os
from pathlib import Path

from . import codec_format

_LIB = None
_LOAD_ERROR: str | None = None
_TOP16_TABLE_CACHE: dict = {}
_TOP16_CODEBOOKS: bytes = (
    Path(__file__).resolve().parent / "data" / "llama_top16_codebooks.bin"
).read_bytes()

_U64 = ctypes.c_ulonglong
_U64P = ctypes.POINTER(ctypes.c_ulonglong)

# (symbol, argtypes, restype, required)
_SIGNATURES = (
    ("kvq_splitzip_bf16_encode", [_U64] * 5, ctypes.c_longlong, True),
    ("kvq_splitzip_bf16_encode_mode", [_U64] * 5 + [ctypes.c_int], ctypes.c_longlong, False),
    ("kvq_splitzip_bf16_decode_fixed6", [_U64] * 10, ctypes.c_longlong, False),
    ("kvq_splitzip_bf16_decode_fixed6_blocks", [_U64] * 11, ctypes.c_longlong, False),
    ("kvq_splitzip_bf16_encode_top16", [_U64] * 6, ctypes.c_longlong, False),
    ("kvq_splitzip_bf16_decode_top16", [_U64] * 11, ctypes.c_longlong, False),
    ("kvq_splitzip_bf16_decode_top16_blocks", [_U64] * 12, ctypes.c_longlong, False),
    # the host block table's address travels as a u64
    ("kvq_splitzip_bf16_decode_top16_host_blocks", [_U64] * 11, ctypes.c_longlong, False),
    ("kvq_splitzip_bf16_decode_fixed6_host_blocks", [_U64] * 10, ctypes.c_longlong, False),
    ("kvq_splitzip_last_error", [], ctypes.c_char_p, True),
    ("kvq_splitzip_top16_paged_workspace_bytes", [_U64, _U64P, _U64], _U64, False),
    ("kvq_splitzip_top16_paged_directory_bytes", [_U64, _U64P, _U64], _U64, False),
    ("kvq_splitzip_top16_paged_presence_bytes", [_U64, _U64P, _U64], _U64, False),
    (
        "kvq_splitzip_top16_build_directory",
        [ctypes.c_void_p, _U64P, _U64P, _U64, _U64, _U64P, ctypes.c_void_p, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_top16_paged",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64, _U64, _U64,
         _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_top16_paged_presence",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64, _U64, _U64,
         _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_top16_paged_probe",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64, _U64, _U64,
         _U64, _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_decode_top16_paged",
        [_U64, _U64P, _U64P, _U64, _U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_top16_paged_noalloc",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    ("kvq_splitzip_top16_noalloc_scratch_bytes", [], _U64, False),
    ("kvq_splitzip_palette_paged_workspace_bytes", [_U64, _U64P, _U64], _U64, False),
    ("kvq_splitzip_top16_decode_attention_workspace_bytes", [_U64] * 3, _U64, False),
    ("kvq_splitzip_exponent_histogram_workspace_bytes", [_U64] * 2, _U64, False),
    ("kvq_splitzip_exponent_histogram_paged", [_U64] * 10, ctypes.c_longlong, False),
    (
        "kvq_splitzip_top16_writeback_paged",
        [_U64, _U64P, _U64P, _U64, _U64, _U64, _U64, _U64, _U64P, _U64P, _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_top16_decode_attention",
        [_U64, _U64, _U64, _U64P, _U64P, _U64, _U64, _U64, _U64, _U64, _U64, _U64, _U64,
         ctypes.c_float, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_mode_paged",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64, _U64,
         ctypes.c_int],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_mode_paged_presence",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64, _U64, _U64P,
         _U64, ctypes.c_int],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_mode_paged_info",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64, _U64P, _U64, _U64,
         ctypes.c_int],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_decode_torchop_paged",
        [_U64, _U64P, _U64P, _U64, _U64, _U64, _U64, _U64, _U64, _U64P, _U64],
        ctypes.c_longlong,
        False,
    ),
    ("kvq_splitzip_torchop_plan_bytes", [], _U64, False),
    ("kvq_splitzip_torchop_workspace_bytes", [_U64, _U64P, _U64], _U64, False),
    (
        "kvq_splitzip_bf16_plan_torchop_paged",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64, _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_encode_torchop_paged",
        [_U64, _U64, _U64, _U64, _U64, _U64P, _U64, _U64, _U64, _U64P, _U64P, _U64, _U64],
        ctypes.c_longlong,
        False,
    ),
    (
        "kvq_splitzip_bf16_decode_mode_paged",
        [_U64, _U64P, _U64P, _U64, _U64, _U64, _U64, _U64, _U64, _U64P, _U64, ctypes.c_int],
        ctypes.c_longlong,
        False,
    ),
)


def _candidate_paths() -> list[str]:
    """``$UNCHAIN_KV_SPLITZIP_LIB``, else the in-tree build, else the loader path."""
    env = os.environ.get("UNCHAIN_KV_SPLITZIP_LIB")
    if env:
        return [env]
    here = Path(__file__).resolve().parent
    return [str(here / "lib" / "libunchain_kv_splitzip_cuda.so"), "libunchain_kv_splitzip_cuda.so"]


def _bind(lib) -> None:
    for name, argtypes, restype, required in _SIGNATURES:
        try:
            fn = getattr(lib, name)
        except AttributeError:
            if required:
                raise
            continue
        fn.argtypes = argtypes
        fn.restype = restype


def _load():
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    errors = []
    for path in _candidate_paths():
        try:
            lib = ctypes.CDLL(path)
        except OSError as exc:
            errors.append(str(exc))
            continue
        # a library without the two mandatory symbols raises AttributeError here,
        # as the reference loader does (src/unchain_kv/splitzip_cuda.py:54-61, 149-150)
        _bind(lib)
        _LIB = lib
        return lib
    _LOAD_ERROR = "; ".join(errors[-2:])
    return None


def available() -> bool:
    return _load() is not None


def load_error() -> str | None:
    _load()
    return _LOAD_ERROR


def _raise_last(lib, default: str):
    message = lib.kvq_splitzip_last_error()
    raise RuntimeError(message.decode() if message else default)


def _is_cuda(tensor) -> bool:
    return getattr(getattr(tensor, "device", None), "type", "") == "cuda"


def _stream_handle(device, torch) -> int:
    """hipStream_t of the current stream of `device`. torch's raw-stream query
    costs ~0.1 us against ~1.9 us for current_stream(device).cuda_stream (measured
    on the MI355X host), a sixth of a small layer's host time per call."""
    raw = getattr(getattr(torch, "_C", None), "_cuda_getCurrentRawStream", None)
    if raw is not None:
        index = device.index if device.index is not None else torch.cuda.current_device()
        return int(raw(index))
    return int(torch.cuda.current_stream(device).cuda_stream)


# ---------------------------------------------------------------------------
# fixed6 / fixed5 (Top-16 fallback)

def encode_bf16(source, out, bits: int = 6) -> int | None:
    lib = _load()
    if lib is None or not _is_cuda(source):
        return None
    if bits not in {5, 6}:
        raise ValueError("splitzip bf16 bits must be 5 or 6")
    import torch

    stream = _stream_handle(source.device, torch)
    encode_mode = getattr(lib, "kvq_splitzip_bf16_encode_mode", None)
    if encode_mode is not None:
        encoded = encode_mode(int(source.data_ptr()), int(out.data_ptr()), int(source.numel()),
                              int(out.numel()), int(stream), int(bits))
    elif bits == 6:
        encoded = lib.kvq_splitzip_bf16_encode(int(source.data_ptr()), int(out.data_ptr()),
                                               int(source.numel()), int(out.numel()), int(stream))
    else:
        return None
    if encoded < 0:
        _raise_last(lib, "splitzip cuda encode failed")
    return int(encoded)


# Block tables of at most this many ids go to the decode in its kernel arguments.
HOST_TABLE_BLOCKS = 256


def _decode_layout(source, out, block_ids, raw_bytes, torch):
    """Validation and geometry of a decode (src/unchain_kv/splitzip_cuda.py:200-230):
    unique in-range block ids, uint8 source and bf16 (2, blocks, ...) target on the
    same CUDA device, both contiguous, raw_bytes an even multiple of 2 * blocks.
    Returns (count_words, block_words, first block, stream handle, contiguous): a
    contiguous ascending run needs no id table. The checks use builtins over the
    id list: with per-id Python checks and a pageable upload a 256-block request
    took 69 us of host time, 31 us this way."""
    if not block_ids or raw_bytes <= 0 or raw_bytes % 2:
        return None
    if not _is_cuda(source) or source.device != getattr(out, "device", None):
        return None
    if source.dtype != torch.uint8 or out.dtype != torch.bfloat16:
        return None
    if not source.is_contiguous() or not out.is_contiguous():
        return None
    if out.dim() < 3 or out.shape[0] != 2:
        return None
    count = len(block_ids)
    lo, hi = min(block_ids), max(block_ids)
    if lo < 0 or hi >= out.shape[1]:
        return None
    start = block_ids[0]
    contiguous = (hi - lo == count - 1 and start == lo
                  and list(block_ids) == list(range(lo, hi + 1)))
    if not contiguous and len(set(block_ids)) != count:
        return None
    count_words = raw_bytes // 2
    if count_words % (2 * count):
        return None
    block_words = count_words // (2 * count)
    return count_words, block_words, start, _stream_handle(out.device, torch), contiguous


def _decode_with_table(lib, host_name, device_name, block_ids, source, out, count_words,
                       block_words, stream, tail, torch):
    """Decode through a non-contiguous block table: in the kernel arguments when the
    library takes the host list (up to HOST_TABLE_BLOCKS ids, tile geometry), else
    from a device copy made asynchronously from pinned memory (recorded on the
    current stream). `tail` = the arguments after the table. Returns the C result,
    or None when no entry point is available."""
    common = (int(source.data_ptr()), int(source.numel()), int(out.data_ptr()), count_words,
              len(block_ids), block_words, int(out.stride(0)), int(out.stride(1)))
    host_decode = getattr(lib, host_name, None)
    if host_decode is not None and len(block_ids) <= HOST_TABLE_BLOCKS:
        table = array.array("q", block_ids)
        copied = host_decode(*common, table.buffer_info()[0], *tail, stream)
        if copied != 0:
            return copied
    device_decode = getattr(lib, device_name, None)
    if device_decode is None:
        return None
    current = torch.cuda.current_stream(out.device)
    ids = torch.tensor(block_ids, dtype=torch.int64, pin_memory=True).to(out.device,
                                                                         non_blocking=True)
    copied = device_decode(*common, block_ids[0], int(ids.data_ptr()), *tail, stream)
    ids.record_stream(current)
    return copied


def decode_fixed6(source, out, block_ids: list[int], raw_bytes: int) -> int | None:
    lib = _load()
    decode = getattr(lib, "kvq_splitzip_bf16_decode_fixed6", None) if lib else None
    if decode is None:
        return None
    import torch

    layout = _decode_layout(source, out, block_ids, raw_bytes, torch)
    if layout is None:
        return None
    count_words, block_words, start, stream, contiguous = layout
    if contiguous:
        copied = decode(int(source.data_ptr()), int(source.numel()), int(out.data_ptr()),
                        count_words, len(block_ids), block_words, int(out.stride(0)),
                        int(out.stride(1)), start, stream)
    else:
        copied = _decode_with_table(lib, "kvq_splitzip_bf16_decode_fixed6_host_blocks",
                                    "kvq_splitzip_bf16_decode_fixed6_blocks", block_ids, source,
                                    out, count_words, block_words, stream, (), torch)
        if copied is None:
            return None
    if copied < 0:
        _raise_last(lib, "splitzip cuda decode failed")
    return int(copied) or None


# ---------------------------------------------------------------------------
# Top-16

def _tables_tensor(codebooks: bytes, device, torch):
    return torch.tensor(list(codec_format.top16_tables(codebooks)), dtype=torch.uint8,
                        device=device)


def _top16_tables(layer_index: int, device, torch):
    """544-byte device table for an embedded layer codebook, cached per
    (device, layer); ``None`` outside the embedded layers
    (src/unchain_kv/splitzip_cuda.py:283-298)."""
    if not 0 <= layer_index < len(_TOP16_CODEBOOKS) // 32:
        return None
    key = (str(device), layer_index)
    cached = _TOP16_TABLE_CACHE.get(key)
    if cached is None:
        cached = _tables_tensor(_TOP16_CODEBOOKS[layer_index * 32:(layer_index + 1) * 32], device,
                                torch)
        _TOP16_TABLE_CACHE[key] = cached
    return cached


def top16_tables_for(codebooks: bytes, device, torch):
    """Device table for an explicit 32-byte codebook, cached per (device, bytes)."""
    codebooks = bytes(codebooks)
    if len(codebooks) != 32:
        raise ValueError("a Top-16 layer codebook is 32 bytes (16 K then 16 V exponents)")
    key = (str(device), codebooks)
    cached = _TOP16_TABLE_CACHE.get(key)
    if cached is None:
        cached = _tables_tensor(codebooks, device, torch)
        _TOP16_TABLE_CACHE[key] = cached
    return cached


def _resolve_tables(layer_index, codebooks, device, torch):
    if codebooks is not None:
        return top16_tables_for(codebooks, device, torch)
    return _top16_tables(layer_index, device, torch)


def encode_top16(source, out, layer_index: int, *, codebooks: bytes | None = None) -> int | None:
    lib = _load()
    encode = getattr(lib, "kvq_splitzip_bf16_encode_top16", None) if lib else None
    if encode is None:
        return None
    if not _is_cuda(source) or source.device != getattr(out, "device", None):
        return None
    import torch

    if source.dtype != torch.bfloat16 or out.dtype != torch.uint8:
        return None
    if not source.is_contiguous() or not out.is_contiguous():
        return None
    tables = _resolve_tables(layer_index, codebooks, source.device, torch)
    if tables is None:
        return None
    stream = _stream_handle(source.device, torch)
    encoded = encode(int(source.data_ptr()), int(out.data_ptr()), int(source.numel()),
                     int(out.numel()), int(tables.data_ptr()), int(stream))
    if encoded < 0:
        _raise_last(lib, "splitzip top16 encode failed")
    return int(encoded) or None


def decode_top16(source, out, block_ids: list[int], raw_bytes: int, layer_index: int, *,
                 codebooks: bytes | None = None) -> int | None:
    lib = _load()
    decode = getattr(lib, "kvq_splitzip_bf16_decode_top16", None) if lib else None
    if decode is None:
        return None
    import torch

    layout = _decode_layout(source, out, block_ids, raw_bytes, torch)
    if layout is None:
        return None
    tables = _resolve_tables(layer_index, codebooks, source.device, torch)
    if tables is None:
        return None
    count_words, block_words, start, stream, contiguous = layout
    if contiguous:
        copied = decode(int(source.data_ptr()), int(source.numel()), int(out.data_ptr()),
                        count_words, len(block_ids), block_words, int(out.stride(0)),
                        int(out.stride(1)), start, int(tables.data_ptr()), stream)
    else:
        copied = _decode_with_table(lib, "kvq_splitzip_bf16_decode_top16_host_blocks",
                                    "kvq_splitzip_bf16_decode_top16_blocks", block_ids, source,
                                    out, count_words, block_words, stream,
                                    (int(tables.data_ptr()),), torch)
        if copied is None:
            return None
    if copied < 0:
        _raise_last(lib, "splitzip top16 decode failed")
    return int(copied) or None


# ---------------------------------------------------------------------------
# batched paged Top-16 (one launch per layer for every request)

class PagedBatch:
    """Block tables of several requests over one paged KV layout.

    ``block_tables[r]`` lists request r's block ids in order; payload r holds the
    K words then the V words of those blocks (the order of
    ``kv_layer[:, block_tables[r]]``). A batch is built once and reused for every
    layer: vLLM gives a request the same block ids in every layer.

    Payload r is placed at ``out_offsets[r]`` of the batch's payload buffer, chosen
    so that its body section starts on a 256-byte boundary (the codes section then
    starts 16-byte aligned too when the block words are a multiple of 16).
    """

    def __init__(self, block_tables, block_words: int, device, torch=None):
        if torch is None:
            import torch
        if not block_tables or any(len(t) == 0 for t in block_tables):
            raise ValueError("every request needs at least one block")
        if block_words <= 0:
            raise ValueError("block_words must be positive")
        self.block_tables = [list(map(int, t)) for t in block_tables]
        self.block_words = int(block_words)
        self.device = device
        flat = [b for t in self.block_tables for b in t]
        if min(flat) < 0:
            raise ValueError("block ids must be non-negative")
        self.ids = torch.tensor(flat, dtype=torch.int64, device=device)
        counts = [len(t) for t in self.block_tables]
        offsets = [0]
        for c in counts:
            offsets.append(offsets[-1] + c)
        self.payload_count = len(counts)
        self.count_words = [2 * c * self.block_words for c in counts]
        self.raw_bytes = [2 * n for n in self.count_words]
        self.encoded_bytes = [codec_format.top16_encoded_size(n) for n in self.count_words]
        out_offsets = []
        end = 0
        for size in self.encoded_bytes:
            start = -(-(end + 5) // 256) * 256 - 5
            out_offsets.append(start)
            end = start + size
        self.out_offsets = out_offsets
        self.out_bytes = end
        self._block_offsets = (ctypes.c_ulonglong * len(offsets))(*offsets)
        self._out_offsets = (ctypes.c_ulonglong * len(out_offsets))(*out_offsets)
        self._encoded = (ctypes.c_ulonglong * len(self.encoded_bytes))(*self.encoded_bytes)
        self.max_block = max(flat)
        self.unique_blocks = len(set(flat)) == len(flat)
        self._palette = {}
        self._workspace = None
        self._runs = None
        self._writeback = {}

    @property
    def runs(self) -> list:
        """Per request: (start, count) when its blocks are one ascending contiguous
        run, else ``None`` (computed once)."""
        if self._runs is None:
            self._runs = [contiguous_run(t) for t in self.block_tables]
        return self._runs

    def writeback_arrays(self, members: tuple):
        """ctypes (offsets, sizes, run starts, run blocks) of ``members`` (cached)."""
        cached = self._writeback.get(members)
        if cached is None:
            runs = [self.runs[r] for r in members]
            if any(run is None for run in runs):
                raise ValueError("writeback needs each request's blocks as one contiguous run")
            k = len(members)
            cached = ((ctypes.c_ulonglong * k)(*(self.out_offsets[r] for r in members)),
                      (ctypes.c_ulonglong * k)(*(self.encoded_bytes[r] for r in members)),
                      (ctypes.c_ulonglong * k)(*(run[0] for run in runs)),
                      (ctypes.c_ulonglong * k)(*(run[1] for run in runs)))
            self._writeback[members] = cached
        return cached

    def _c_array(self, values, own, own_array):
        """ctypes u64 array of `values` (the batch's own array when it is the same list)."""
        if values is own:
            return own_array
        return (ctypes.c_ulonglong * self.payload_count)(*map(int, values))

    @property
    def total_raw_bytes(self) -> int:
        return sum(self.raw_bytes)

    @property
    def total_encoded_bytes(self) -> int:
        return sum(self.encoded_bytes)

    def workspace_bytes(self) -> int:
        lib = _load()
        query = getattr(lib, "kvq_splitzip_top16_paged_workspace_bytes", None) if lib else None
        if query is None:
            raise RuntimeError(f"splitzip HIP library unavailable: {load_error()}")
        return int(query(self.block_words, self._block_offsets, self.payload_count))

    def new_payload_buffer(self, torch=None):
        if torch is None:
            import torch
        return torch.empty(self.out_bytes, dtype=torch.uint8, device=self.device)

    def new_workspace(self, torch=None):
        if torch is None:
            import torch
        return torch.empty(max(self.workspace_bytes(), 16), dtype=torch.uint8,
                           device=self.device)

    def workspace(self, torch=None):
        """This batch's own encode workspace, made by new_workspace on first use and
        kept, so that recurring batches allocate it once: calls with the same batch
        on one stream reuse it (calls that may overlap on different streams need
        workspaces of their own)."""
        if self._workspace is None:
            self._workspace = self.new_workspace(torch)
        return self._workspace

    def directory_bytes(self) -> int:
        """Bytes of the batch's escape directory (0 when its block geometry has none:
        block words not a multiple of 1024)."""
        lib = _load()
        query = getattr(lib, "kvq_splitzip_top16_paged_directory_bytes", None) if lib else None
        if query is None:
            raise RuntimeError(f"splitzip HIP library unavailable: {load_error()}")
        return int(query(self.block_words, self._block_offsets, self.payload_count))

    def new_directory(self, torch=None):
        """Device buffer for the escape directory, or None when the batch has none."""
        if torch is None:
            import torch
        size = self.directory_bytes()
        return torch.empty(size, dtype=torch.uint8, device=self.device) if size else None

    def presence_bytes(self) -> int:
        """Bytes of the batch's high-byte presence masks (32 per 4096-word tile of
        each plane; 0 when block words are not a multiple of 1024)."""
        lib = _load()
        query = getattr(lib, "kvq_splitzip_top16_paged_presence_bytes", None) if lib else None
        if query is None:
            raise RuntimeError(f"splitzip HIP library unavailable: {load_error()}")
        return int(query(self.block_words, self._block_offsets, self.payload_count))

    def new_presence(self, torch=None):
        """Device buffer for the presence masks, or None when the batch has none."""
        if torch is None:
            import torch
        size = self.presence_bytes()
        return torch.empty(size, dtype=torch.uint8, device=self.device) if size else None

    PALETTE_INFO_BYTES = 512

    def new_palette_info(self, torch=None):
        """Device buffer for one 512-byte palette record per request (written by a
        probe encode: ``encode_top16_paged(presence=..., palette_info=...)``)."""
        if torch is None:
            import torch
        return torch.empty(self.PALETTE_INFO_BYTES * self.payload_count, dtype=torch.uint8,
                           device=self.device)

    def presence_first(self, members) -> list[int]:
        """Index of the first presence mask of each request in ``members`` (masks
        of request r follow those of requests 0 .. r-1, one per 4096-word tile of
        each plane)."""
        firsts, at = [], 0
        for n in self.count_words:
            firsts.append(at)
            at += 2 * (-(-(n // 2) // 4096))
        return [firsts[r] for r in members]

    def payload(self, out, r: int):
        return out[self.out_offsets[r]:self.out_offsets[r] + self.encoded_bytes[r]]

    def palette_layout(self, bits: int) -> tuple[list[int], list[int], int]:
        """(offsets, encoded sizes, buffer bytes) of the batch's fixed6 (bits 6) or
        fixed5 (bits 5) payloads; each payload's low-byte section starts on a
        256-byte boundary."""
        cached = self._palette.get(bits)
        if cached is None:
            header = codec_format.palette_header_bytes(bits)
            sizes = [codec_format.palette_encoded_size(n, bits) for n in self.count_words]
            offsets, end = [], 0
            for size in sizes:
                start = -(-(end + header) // 256) * 256 - header
                offsets.append(start)
                end = start + size
            cached = (offsets, sizes, end, (ctypes.c_ulonglong * len(offsets))(*offsets),
                      (ctypes.c_ulonglong * len(sizes))(*sizes))
            self._palette[bits] = cached
        return cached[0], cached[1], cached[2]

    def palette_workspace_bytes(self) -> int:
        lib = _load()
        query = getattr(lib, "kvq_splitzip_palette_paged_workspace_bytes", None) if lib else None
        if query is None:
            raise RuntimeError(f"splitzip HIP library unavailable: {load_error()}")
        return int(query(self.block_words, self._block_offsets, self.payload_count))

    def new_palette_buffer(self, bits: int, torch=None):
        if torch is None:
            import torch
        return torch.empty(self.palette_layout(bits)[2], dtype=torch.uint8, device=self.device)

    def new_palette_workspace(self, torch=None):
        if torch is None:
            import torch
        return torch.empty(max(self.palette_workspace_bytes(), 16), dtype=torch.uint8,
                           device=self.device)


def _paged_layout_ok(kv_layer, batch: PagedBatch, torch) -> bool:
    if not _is_cuda(kv_layer) or kv_layer.dtype != torch.bfloat16:
        return False
    shape = kv_layer.shape
    if len(shape) < 3 or shape[0] != 2 or not kv_layer.is_contiguous():
        return False
    block_words = 1
    for extent in shape[2:]:
        block_words *= extent
    return block_words == batch.block_words and batch.max_block < shape[1]


def _payloads_fit(source, src_offsets, encoded_bytes, batch: PagedBatch) -> bool:
    if len(src_offsets) != batch.payload_count or len(encoded_bytes) != batch.payload_count:
        return False
    size = source.numel() if hasattr(source, "numel") and callable(source.numel) else source.size
    return all(o + e <= size for o, e in zip(src_offsets, encoded_bytes))


def _byte_buffer_ok(buf, device, nbytes: int, torch) -> bool:
    """A contiguous uint8 tensor on ``device`` holding at least ``nbytes`` bytes."""
    return buf is not None and buf.dtype == torch.uint8 and buf.is_contiguous() and \
        buf.device == device and buf.numel() >= nbytes


def _directory_ptr(directory, batch: PagedBatch, torch) -> int | None:
    """Device address of an escape directory (0 for none); None when unusable."""
    if directory is None:
        return 0
    if directory.dtype != torch.uint8 or not directory.is_contiguous() or \
            directory.device != batch.ids.device or directory.numel() < batch.directory_bytes():
        return None
    return int(directory.data_ptr())


def encode_top16_paged(kv_layer, batch: PagedBatch, out, workspace, layer_index: int = -1, *,
                       codebooks: bytes | None = None, tables=None,
                       directory=None, presence=None, palette_info=None) -> int | None:
    """Gather + Top-16 encode every request of ``batch`` from one paged layer
    ``(2, num_blocks, ...)`` into ``out`` (a ``batch.out_bytes`` uint8 buffer).
    With ``directory`` (``batch.new_directory()``) the encoder also writes the
    escape directory that lets ``decode_top16_paged`` apply escapes without a
    second pass; with ``presence`` (``batch.new_presence()``) it writes the
    high-byte presence masks that let ``encode_bf16_paged`` re-encode an
    overflowed request without a presence pass. ``palette_info``
    (``batch.new_palette_info()``, with ``presence``): a probe encode of a layer
    that overflowed before; it also writes every request's fixed6/fixed5 palette
    record (``encode_bf16_paged(palette_info=...)`` then needs no presence or
    reduce pass) and leaves an overflowed payload's escape slots unplaced (its
    header, body and codes are written; it is re-encoded anyway). Returns the total
    encoded bytes or ``None`` when the codec declines."""
    if palette_info is not None and presence is None:
        raise ValueError("palette_info needs presence")
    if workspace is None:
        raise ValueError("encode_top16_paged needs a workspace (batch.workspace())")
    lib = _load()
    name = "kvq_splitzip_bf16_encode_top16_paged" + (
        "_probe" if palette_info is not None else "_presence" if presence is not None else "")
    encode = getattr(lib, name, None) if lib else None
    if encode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    if out.dtype != torch.uint8 or not out.is_contiguous() or out.device != kv_layer.device:
        return None
    if tables is None:
        tables = _resolve_tables(layer_index, codebooks, kv_layer.device, torch)
    dir_ptr = _directory_ptr(directory, batch, torch)
    if tables is None or dir_ptr is None:
        return None
    if not _byte_buffer_ok(workspace, kv_layer.device, 1, torch):
        return None
    extra = ()
    if presence is not None:
        if presence.dtype != torch.uint8 or not presence.is_contiguous() or \
                presence.device != kv_layer.device or presence.numel() < batch.presence_bytes() \
                or batch.presence_bytes() == 0:
            return None
        extra = (int(presence.data_ptr()),)
    if palette_info is not None:
        if palette_info.dtype != torch.uint8 or not palette_info.is_contiguous() or \
                palette_info.device != kv_layer.device or \
                palette_info.numel() < PagedBatch.PALETTE_INFO_BYTES * batch.payload_count:
            return None
        extra += (int(palette_info.data_ptr()),)
    stream = _stream_handle(kv_layer.device, torch)
    encoded = encode(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                     batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                     batch.payload_count, int(out.data_ptr()), batch._out_offsets,
                     int(out.numel()), int(tables.data_ptr()), int(workspace.data_ptr()),
                     int(workspace.numel()), dir_ptr, *extra, int(stream))
    if encoded < 0:
        _raise_last(lib, "splitzip top16 paged encode failed")
    return int(encoded) or None


def encode_top16_paged_noalloc(kv_layer, batch: PagedBatch, out, layer_index: int = -1, *,
                               codebooks: bytes | None = None, tables=None,
                               directory=None) -> int | None:
    """``encode_top16_paged`` without a workspace argument and without any
    allocation by the library: its scratch is a fixed array of
    ``noalloc_scratch_bytes()`` bytes per GPU, shared by every call on that GPU
    (calls that overlap on one GPU race). Raises ``RuntimeError`` for a batch
    that needs more scratch than that."""
    lib = _load()
    encode = getattr(lib, "kvq_splitzip_bf16_encode_top16_paged_noalloc", None) if lib else None
    if encode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    if out.dtype != torch.uint8 or not out.is_contiguous() or out.device != kv_layer.device:
        return None
    if tables is None:
        tables = _resolve_tables(layer_index, codebooks, kv_layer.device, torch)
    dir_ptr = _directory_ptr(directory, batch, torch)
    if tables is None or dir_ptr is None:
        return None
    stream = _stream_handle(kv_layer.device, torch)
    encoded = encode(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                     batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                     batch.payload_count, int(out.data_ptr()), batch._out_offsets,
                     int(out.numel()), int(tables.data_ptr()), dir_ptr, int(stream))
    if encoded < 0:
        _raise_last(lib, "splitzip top16 paged encode (no allocation) failed")
    return int(encoded) or None


def noalloc_scratch_bytes() -> int:
    """Bytes of the library's fixed per-GPU scratch for encode_top16_paged_noalloc."""
    lib = _load()
    query = getattr(lib, "kvq_splitzip_top16_noalloc_scratch_bytes", None) if lib else None
    if query is None:
        raise RuntimeError(f"splitzip HIP library unavailable: {load_error()}")
    return int(query())


def decode_top16_paged(source, src_offsets, encoded_bytes, kv_layer, batch: PagedBatch,
                       layer_index: int = -1, *, codebooks: bytes | None = None,
                       tables=None, directory=None) -> int | None:
    """Decode payload r (``source[src_offsets[r]:][:encoded_bytes[r]]``) and scatter
    it into ``batch.block_tables[r]`` of the paged layer ``kv_layer``; one launch
    for every request. ``directory``: the escape directory written by the encode of
    these payloads (for a batch with the same block counts), or built on the host
    by ``build_directory``; the decode is then one kernel. Returns the total raw
    bytes written or ``None``."""
    lib = _load()
    decode = getattr(lib, "kvq_splitzip_bf16_decode_top16_paged", None) if lib else None
    if decode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch) or not batch.unique_blocks:
        return None
    if source.dtype != torch.uint8 or not source.is_contiguous() or source.device != kv_layer.device:
        return None
    if not _payloads_fit(source, src_offsets, encoded_bytes, batch):
        return None
    if tables is None:
        tables = _resolve_tables(layer_index, codebooks, kv_layer.device, torch)
    dir_ptr = _directory_ptr(directory, batch, torch)
    if tables is None or dir_ptr is None:
        return None
    offs = batch._c_array(src_offsets, batch.out_offsets, batch._out_offsets)
    encs = batch._c_array(encoded_bytes, batch.encoded_bytes, batch._encoded)
    stream = _stream_handle(kv_layer.device, torch)
    copied = decode(int(source.data_ptr()), offs, encs, batch.payload_count,
                    int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                    batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                    int(tables.data_ptr()), dir_ptr, int(stream))
    if copied < 0:
        _raise_last(lib, "splitzip top16 paged decode failed")
    return int(copied) or None


def build_directory(host_payloads, src_offsets, encoded_bytes, batch: PagedBatch):
    """Escape directory of Top-16 payloads held in host memory (a writable uint8
    numpy array or CPU tensor; payload r at ``src_offsets[r]``, ``encoded_bytes[r]``
    long, of ``batch``'s block counts), as a uint8 numpy array to copy to the
    device with the payloads. Each mode-5 payload's escape list is sorted by
    position in place (the decode does not depend on its order). ``None`` when the
    batch's geometry has no directory or a size does not match."""
    import numpy as np

    lib = _load()
    build = getattr(lib, "kvq_splitzip_top16_build_directory", None) if lib else None
    if build is None:
        return None
    buf = host_payloads.numpy() if hasattr(host_payloads, "numpy") else host_payloads
    if buf.dtype != np.uint8 or not buf.flags["C_CONTIGUOUS"] or not buf.flags["WRITEABLE"]:
        raise ValueError("host payloads must be a writable contiguous uint8 array")
    if not _payloads_fit(buf.reshape(-1), src_offsets, encoded_bytes, batch):
        return None
    size = batch.directory_bytes()
    if not size:
        return None
    out = np.empty(size, dtype=np.uint8)
    offs = batch._c_array(src_offsets, batch.out_offsets, batch._out_offsets)
    encs = batch._c_array(encoded_bytes, batch.encoded_bytes, batch._encoded)
    got = build(buf.ctypes.data, offs, encs, batch.payload_count, batch.block_words,
                batch._block_offsets, out.ctypes.data, size)
    return out if got == size else None


# ---------------------------------------------------------------------------
# batched paged fixed6 / fixed5 (the Top-16 overflow fallback, one launch per layer)

def encode_bf16_paged(kv_layer, batch: PagedBatch, out, workspace, bits: int = 6, *,
                      presence=None, presence_first=None, palette_info=None,
                      info_first=None) -> int | None:
    """Gather + fixed6 (bits 6) or fixed5 (bits 5) encode of every request of
    ``batch``; payload r goes to ``batch.palette_layout(bits)[0][r]`` of ``out``.
    ``presence`` / ``presence_first``: the high-byte presence masks a Top-16
    encode of the same blocks wrote (``encode_top16_paged(presence=...)``) and the
    index of request r's first mask there (``PagedBatch.presence_first`` of that
    batch); the encode then skips its own presence pass. ``palette_info`` /
    ``info_first``: the palette records a probe encode of the same blocks wrote
    (``encode_top16_paged(presence=..., palette_info=...)``) and the index of
    request r's record there; the encode is then one pass (``workspace`` unused).
    Returns the total encoded bytes or ``None`` when the codec declines."""
    if bits not in {5, 6}:
        raise ValueError("splitzip bf16 bits must be 5 or 6")
    if (presence is None) != (presence_first is None):
        raise ValueError("presence and presence_first go together")
    if (palette_info is None) != (info_first is None):
        raise ValueError("palette_info and info_first go together")
    if palette_info is not None:
        return _encode_bf16_paged_info(kv_layer, batch, out, bits, palette_info, info_first)
    if workspace is None:
        raise ValueError("encode_bf16_paged needs a workspace (batch.new_palette_workspace()) "
                         "unless palette_info is given")
    lib = _load()
    name = "kvq_splitzip_bf16_encode_mode_paged" + ("_presence" if presence is not None else "")
    encode = getattr(lib, name, None) if lib else None
    if encode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    if out.dtype != torch.uint8 or not out.is_contiguous() or out.device != kv_layer.device:
        return None
    if not _byte_buffer_ok(workspace, kv_layer.device, 1, torch):
        return None
    batch.palette_layout(bits)
    offs = batch._palette[bits][3]
    extra = ()
    if presence is not None:
        if presence.dtype != torch.uint8 or not presence.is_contiguous() or \
                presence.device != kv_layer.device or len(presence_first) != batch.payload_count:
            return None
        # every request's masks must lie inside the buffer
        for first, n in zip(presence_first, batch.count_words):
            if first < 0 or 32 * (first + 2 * (-(-(n // 2) // 4096))) > presence.numel():
                return None
        extra = (int(presence.data_ptr()),
                 (ctypes.c_ulonglong * batch.payload_count)(*map(int, presence_first)))
    stream = _stream_handle(kv_layer.device, torch)
    encoded = encode(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                     batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                     batch.payload_count, int(out.data_ptr()), offs, int(out.numel()),
                     int(workspace.data_ptr()), int(workspace.numel()), *extra, int(stream),
                     int(bits))
    if encoded < 0:
        _raise_last(lib, "splitzip palette paged encode failed")
    return int(encoded) or None


def _encode_bf16_paged_info(kv_layer, batch, out, bits, palette_info, info_first):
    lib = _load()
    encode = getattr(lib, "kvq_splitzip_bf16_encode_mode_paged_info", None) if lib else None
    if encode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    if out.dtype != torch.uint8 or not out.is_contiguous() or out.device != kv_layer.device:
        return None
    if palette_info.dtype != torch.uint8 or not palette_info.is_contiguous() or \
            palette_info.device != kv_layer.device or len(info_first) != batch.payload_count:
        return None
    records = palette_info.numel() // PagedBatch.PALETTE_INFO_BYTES
    batch.palette_layout(bits)
    offs = batch._palette[bits][3]
    firsts = (ctypes.c_ulonglong * batch.payload_count)(*map(int, info_first))
    stream = _stream_handle(kv_layer.device, torch)
    encoded = encode(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                     batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                     batch.payload_count, int(out.data_ptr()), offs, int(out.numel()),
                     int(palette_info.data_ptr()), firsts, records, int(stream), int(bits))
    if encoded < 0:
        _raise_last(lib, "splitzip palette paged encode (probe palettes) failed")
    return int(encoded) or None


def decode_bf16_paged(source, src_offsets, encoded_bytes, kv_layer, batch: PagedBatch,
                      bits: int = 6) -> int | None:
    """Decode fixed6 (bits 6) or fixed5 (bits 5) payload r
    (``source[src_offsets[r]:][:encoded_bytes[r]]``) and scatter it into
    ``batch.block_tables[r]``; one launch for every request."""
    if bits not in {5, 6}:
        raise ValueError("splitzip bf16 bits must be 5 or 6")
    lib = _load()
    decode = getattr(lib, "kvq_splitzip_bf16_decode_mode_paged", None) if lib else None
    if decode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch) or not batch.unique_blocks:
        return None
    if source.dtype != torch.uint8 or not source.is_contiguous() or source.device != kv_layer.device:
        return None
    if not _payloads_fit(source, src_offsets, encoded_bytes, batch):
        return None
    layout = batch._palette.get(bits)
    if layout is not None and src_offsets is layout[0] and encoded_bytes is layout[1]:
        offs, encs = layout[3], layout[4]
    else:
        offs = batch._c_array(src_offsets, None, None)
        encs = batch._c_array(encoded_bytes, None, None)
    stream = _stream_handle(kv_layer.device, torch)
    copied = decode(int(source.data_ptr()), offs, encs, batch.payload_count,
                    int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                    batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                    int(stream), int(bits))
    if copied < 0:
        _raise_last(lib, "splitzip palette paged decode failed")
    return int(copied) or None


def decode_torchop_paged(source, src_offsets, encoded_bytes, kv_layer,
                         batch: PagedBatch) -> int | None:
    """Decode the reference connector's torch-op payloads (modes 0, 1, 2: palette,
    nibble planes, sign/magnitude; src/unchain_kv/vllm_connector.py:5168-5252)
    ``source[src_offsets[r]:][:encoded_bytes[r]]`` and scatter payload r into
    ``batch.block_tables[r]``; modes may be mixed. A payload whose header does not
    match its size is left unapplied. Returns the total raw bytes or ``None``."""
    lib = _load()
    decode = getattr(lib, "kvq_splitzip_bf16_decode_torchop_paged", None) if lib else None
    if decode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch) or not batch.unique_blocks:
        return None
    if source.dtype != torch.uint8 or not source.is_contiguous() or source.device != kv_layer.device:
        return None
    if not _payloads_fit(source, src_offsets, encoded_bytes, batch):
        return None
    offs = batch._c_array(src_offsets, None, None)
    encs = batch._c_array(encoded_bytes, None, None)
    stream = _stream_handle(kv_layer.device, torch)
    copied = decode(int(source.data_ptr()), offs, encs, batch.payload_count,
                    int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                    batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                    int(stream))
    if copied < 0:
        _raise_last(lib, "splitzip torch-op paged decode failed")
    return int(copied) or None


# ---------------------------------------------------------------------------
# torch-op encode (the sender's formats for small requests)

TORCHOP_PLAN_BYTES = 64


def plan_torchop_paged(kv_layer, batch: PagedBatch, plans=None):
    """Queue the plan of the reference connector's torch-op encode of every request
    of ``batch`` (src/unchain_kv/vllm_connector.py:3204-3343: sign/magnitude, else
    the high-byte palette, else the nibble planes, else none). Returns the device
    tensor of 64-byte plan records (``plans`` when given), or ``None`` when the
    library declines; ``read_torchop_plans`` turns a host copy into sizes."""
    lib = _load()
    plan = getattr(lib, "kvq_splitzip_bf16_plan_torchop_paged", None) if lib else None
    if plan is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    size = int(lib.kvq_splitzip_torchop_workspace_bytes(batch.block_words, batch._block_offsets,
                                                        batch.payload_count))
    if size == 0:
        return None
    if plans is None:
        plans = torch.empty(TORCHOP_PLAN_BYTES * batch.payload_count, dtype=torch.uint8,
                            device=kv_layer.device)
    elif plans.dtype != torch.uint8 or plans.numel() < TORCHOP_PLAN_BYTES * batch.payload_count \
            or not plans.is_contiguous() or plans.device != kv_layer.device:
        return None
    workspace = torch.empty(size, dtype=torch.uint8, device=kv_layer.device)
    stream = _stream_handle(kv_layer.device, torch)
    got = plan(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
               batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
               batch.payload_count, int(workspace.data_ptr()), size, int(plans.data_ptr()),
               int(stream))
    if got < 0:
        _raise_last(lib, "splitzip torch-op plan failed")
    # (the workspace goes back to torch's caching allocator on return: a later
    # allocation reuses it only for work queued on this stream after the plan's)
    return plans if got else None


def read_torchop_plans(host_plans) -> list[tuple[int, int]]:
    """(mode, encoded bytes) per request from a host copy of the plan records; mode
    255 and 0 bytes for a request no torch-op format compresses."""
    import numpy as np

    raw = np.asarray(host_plans, dtype=np.uint8).reshape(-1, TORCHOP_PLAN_BYTES)
    sizes = raw[:, 48:56].copy().view(np.uint64).reshape(-1)
    return [(int(raw[r, 36]), int(sizes[r])) for r in range(raw.shape[0])]


def encode_torchop_paged(kv_layer, batch: PagedBatch, plans, out, out_offsets,
                         encoded_bytes) -> int | None:
    """Write request r's torch-op payload, as the reference's encoder writes it, to
    ``out[out_offsets[r]:][:encoded_bytes[r]]`` per its plan (``encoded_bytes[r]``
    from ``read_torchop_plans``; 0 skips the request). Returns the total encoded
    bytes, or ``None`` when the library declines."""
    lib = _load()
    encode = getattr(lib, "kvq_splitzip_bf16_encode_torchop_paged", None) if lib else None
    if encode is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    if out.dtype != torch.uint8 or not out.is_contiguous() or out.device != kv_layer.device:
        return None
    if plans.numel() < TORCHOP_PLAN_BYTES * batch.payload_count or plans.device != out.device:
        return None
    if len(out_offsets) != batch.payload_count or len(encoded_bytes) != batch.payload_count:
        return None
    offs = batch._c_array(out_offsets, None, None)
    encs = batch._c_array(encoded_bytes, None, None)
    stream = _stream_handle(kv_layer.device, torch)
    got = encode(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
                 batch.block_words, int(batch.ids.data_ptr()), batch._block_offsets,
                 batch.payload_count, int(plans.data_ptr()), int(out.data_ptr()), offs, encs,
                 int(out.numel()), int(stream))
    if got < 0:
        _raise_last(lib, "splitzip torch-op encode failed")
    return int(got) if got or not any(encoded_bytes) else None


# ---------------------------------------------------------------------------
# fused Top-16 decode + decode attention

def decode_attention_workspace_bytes(batch: int, kv_heads: int, max_context: int) -> int:
    """Bytes of the workspace decode_attention_top16 uses (split partials)."""
    lib = _load()
    if lib is None or not hasattr(lib, "kvq_splitzip_top16_decode_attention_workspace_bytes"):
        raise RuntimeError(f"HIP codec library not loaded: {load_error()}")
    return int(lib.kvq_splitzip_top16_decode_attention_workspace_bytes(batch, kv_heads,
                                                                        max_context))


def decode_attention_top16(q, payloads, payload_offsets, context_tokens, kv_heads: int,
                           layer_index: int = -1, *, block_tokens: int = 16,
                           codebooks: bytes | None = None, tables=None,
                           scale: float | None = None, out=None, workspace=None):
    """Attention of one query token per sequence over Top-16 packed KV, decoded
    in LDS (no bf16 KV is written). ``q`` is (batch, q_heads, 128) bf16 with
    q_heads = 4 * kv_heads; sequence r's payload starts at ``payload_offsets[r]``
    of the uint8 tensor ``payloads`` and is the encoder's payload of its block
    table in token order (ceil(context_tokens[r] / block_tokens) whole blocks),
    words ordered [token][kv head][dim] for the K plane, then the V plane; the
    first ``context_tokens[r]`` tokens are attended. Returns the (batch, q_heads,
    128) bf16 output, or ``None`` when the kernel declines."""
    lib = _load()
    attend = getattr(lib, "kvq_splitzip_top16_decode_attention", None) if lib else None
    if attend is None:
        return None
    import torch

    if not _is_cuda(q) or q.dtype != torch.bfloat16 or not q.is_contiguous() or q.dim() != 3:
        return None
    if payloads.dtype != torch.uint8 or not payloads.is_contiguous() or payloads.device != q.device:
        return None
    batch, q_heads, head_dim = q.shape
    if len(payload_offsets) != batch or len(context_tokens) != batch:
        return None
    if block_tokens <= 0:
        return None
    for off, ctx in zip(payload_offsets, context_tokens):
        span = -(-int(ctx) // block_tokens) * block_tokens
        n = 2 * span * kv_heads * head_dim
        if int(off) < 0 or int(off) + codec_format.top16_encoded_size(n) > payloads.numel():
            return None
    if tables is None:
        tables = _resolve_tables(layer_index, codebooks, q.device, torch)
    if tables is None:
        return None
    if scale is None:
        scale = head_dim ** -0.5
    if out is None:
        out = torch.empty_like(q)
    elif out.dtype != torch.bfloat16 or not out.is_contiguous() or out.shape != q.shape or \
            out.device != q.device:
        return None
    max_ctx = max(int(c) for c in context_tokens)
    need = int(lib.kvq_splitzip_top16_decode_attention_workspace_bytes(batch, kv_heads, max_ctx))
    if not _byte_buffer_ok(workspace, q.device, need, torch):
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    offs = (ctypes.c_ulonglong * batch)(*map(int, payload_offsets))
    ctxs = (ctypes.c_ulonglong * batch)(*map(int, context_tokens))
    stream = _stream_handle(q.device, torch)
    got = attend(int(q.data_ptr()), int(out.data_ptr()), int(payloads.data_ptr()), offs, ctxs,
                 int(block_tokens), batch, q_heads, kv_heads, head_dim, int(tables.data_ptr()),
                 int(workspace.data_ptr()), int(workspace.numel()), float(scale), int(stream))
    if got < 0:
        _raise_last(lib, "splitzip top16 decode attention failed")
    return out if got else None


# ---------------------------------------------------------------------------
# codec writeback (payloads moved into the sender's own blocks)

def contiguous_run(block_ids) -> tuple[int, int] | None:
    """(start, count) when ``block_ids`` is one ascending run start, start + 1, ...
    (the only layout the reference writes back into, vllm_connector.py:3479-3488),
    else ``None``."""
    ids = [int(b) for b in block_ids]
    if not ids or any(b != ids[0] + i for i, b in enumerate(ids)):
        return None
    return ids[0], len(ids)


def writeback_top16_paged(payloads, batch: PagedBatch, kv_layer, members, *, status=None):
    """Codec writeback (src/unchain_kv/vllm_connector.py:3460-3563): for each r in
    ``members``, moves Top-16 payload r of ``batch`` (``batch.out_offsets[r]`` of
    ``payloads``) into request r's own blocks of ``kv_layer``: its first bytes into
    the K-plane run of the request's blocks, the rest into the V-plane run (the
    reference's two segment copies). Every member's block table must be one
    ascending contiguous run (``contiguous_run``). A payload whose mode byte is not
    5 (an overflow) is not written, so its blocks stay intact for the fallback
    encode. Returns ``(bytes, status)``: the bytes of the members' payloads (0 when
    the library declines: runs that overlap each other or the payload buffer) and a
    device uint8 tensor with each member's mode byte."""
    lib = _load()
    move = getattr(lib, "kvq_splitzip_top16_writeback_paged", None) if lib else None
    if move is None:
        raise RuntimeError(f"HIP codec library not loaded: {load_error()}")
    import torch

    members = tuple(int(r) for r in members)
    if not members:
        raise ValueError("no payloads to write back")
    if not _paged_layout_ok(kv_layer, batch, torch):
        raise ValueError("kv_layer is not a contiguous bf16 (2, num_blocks, ...) layer of this batch")
    if payloads.dtype != torch.uint8 or not payloads.is_contiguous() or \
            payloads.device != kv_layer.device or payloads.numel() < batch.out_bytes:
        raise ValueError("payloads must be the batch's contiguous uint8 payload buffer")
    offs, sizes, starts, counts = batch.writeback_arrays(members)
    k = len(members)
    if status is None:
        status = torch.empty(k, dtype=torch.uint8, device=kv_layer.device)
    elif status.dtype != torch.uint8 or status.numel() < k or status.device != kv_layer.device:
        raise ValueError("status must be a device uint8 tensor with one byte per member")
    stream = _stream_handle(kv_layer.device, torch)
    got = move(int(payloads.data_ptr()), offs, sizes, k, int(kv_layer.data_ptr()),
               int(kv_layer.stride(0)), int(kv_layer.stride(1)), batch.block_words, starts,
               counts, int(status.data_ptr()), int(stream))
    if got < 0:
        _raise_last(lib, "splitzip top16 writeback failed")
    return int(got), status


# ---------------------------------------------------------------------------
# exponent histograms (codebook fitting)

def exponent_histogram_workspace_bytes(block_count: int, block_words: int) -> int:
    lib = _load()
    if lib is None or not hasattr(lib, "kvq_splitzip_exponent_histogram_workspace_bytes"):
        raise RuntimeError(f"HIP codec library not loaded: {load_error()}")
    return int(lib.kvq_splitzip_exponent_histogram_workspace_bytes(block_count, block_words))


def exponent_histogram_paged(kv_layer, batch: PagedBatch, *, workspace=None, counts=None):
    """(2, 256) int64 device tensor: per K/V plane, the count of every bf16 exponent
    (bits 7..14) over all blocks of ``batch`` in the paged layer ``kv_layer`` (what
    the reference's exponent trace bins with torch.bincount per plane,
    src/unchain_kv/vllm_connector.py:2871-2904). ``None`` when the kernel declines."""
    lib = _load()
    hist = getattr(lib, "kvq_splitzip_exponent_histogram_paged", None) if lib else None
    if hist is None:
        return None
    import torch

    if not _paged_layout_ok(kv_layer, batch, torch):
        return None
    count = len(batch.ids)
    need = int(lib.kvq_splitzip_exponent_histogram_workspace_bytes(count, batch.block_words))
    if not _byte_buffer_ok(workspace, kv_layer.device, need, torch):
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=kv_layer.device)
    if counts is None:
        counts = torch.empty((2, 256), dtype=torch.int64, device=kv_layer.device)
    stream = _stream_handle(kv_layer.device, torch)
    got = hist(int(kv_layer.data_ptr()), int(kv_layer.stride(0)), int(kv_layer.stride(1)),
               batch.block_words, int(batch.ids.data_ptr()), count, int(counts.data_ptr()),
               int(workspace.data_ptr()), int(workspace.numel()), int(stream))
    if got < 0:
        _raise_last(lib, "splitzip exponent histogram failed")
    return counts if got else None


def fit_top16_codebook_paged(kv_layer, batch: PagedBatch) -> bytes | None:
    """The layer's 32-byte Top-16 codebook (16 K exponents, then 16 V) fit on the
    GPU histogram of ``batch``'s blocks with the reference's rule: the 16 most
    frequent exponents by (-count, value) (scripts/extract_llama_top16_codebooks.py
    :15-60). ``None`` when a plane has fewer than 16 distinct exponents."""
    from . import codebooks as cb

    counts = exponent_histogram_paged(kv_layer, batch)
    if counts is None:
        return None
    k, v = counts.cpu().tolist()
    try:
        return cb.fit_layer_codebook(k, v)
    except ValueError:
        return None
