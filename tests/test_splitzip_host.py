"""Host-side behaviour of the drop-in ``splitzip_cuda`` module, with no GPU.

The first tests restate tests/test_splitzip_cuda.py:10-90, 187-336 of the
reference: a fake library records the exact positional C-ABI arguments, fake
tensors stand in for torch. The argument tuples come from
tests/golden/kat_abi_calls.json. The last tests load the real HIP library and
check that it exports every symbol declared in include/unchain_kv_splitzip.h.
"""

import ctypes
import json
import re
import sys
from pathlib import Path
from types import SimpleNamespace
from unittest.mock import patch

import pytest

from unchainkv_amd import splitzip_cuda

ROOT = Path(__file__).resolve().parents[1]


class FakeTensor:
    def __init__(self, ptr, shape, stride, dtype, device):
        self._ptr = ptr
        self.shape = tuple(shape)
        self._stride = tuple(stride)
        self.dtype = dtype
        self.device = device

    def data_ptr(self):
        return self._ptr

    def numel(self):
        result = 1
        for size in self.shape:
            result *= size
        return result

    def dim(self):
        return len(self.shape)

    def stride(self, dim):
        return self._stride[dim]

    def is_contiguous(self):
        return True


@pytest.fixture(scope="module")
def abi():
    return json.loads((ROOT / "tests" / "golden" / "kat_abi_calls.json").read_text())


def _fake_torch(stream, **extra):
    return SimpleNamespace(
        uint8=extra.pop("uint8"),
        bfloat16=extra.pop("bfloat16"),
        cuda=SimpleNamespace(current_stream=lambda _device: stream),
        **extra,
    )


def test_top16_layer_bound_follows_codebook_count():
    layers = len(splitzip_cuda._TOP16_CODEBOOKS) // 32
    assert layers == 32
    assert splitzip_cuda._top16_tables(layers, "cuda", object()) is None
    assert splitzip_cuda._top16_tables(-1, "cuda", object()) is None


def test_top16_wrappers_pass_static_tables(abi):
    encode_calls, decode_calls = [], []

    class FakeLib:
        def kvq_splitzip_bf16_encode_top16(self, *args):
            encode_calls.append(args)
            return 13

        def kvq_splitzip_bf16_decode_top16(self, *args):
            decode_calls.append(args)
            return 16

    device = SimpleNamespace(type="cuda")
    uint8, bfloat16 = object(), object()
    e, d = abi["encode_top16"], abi["decode_top16"]
    source = FakeTensor(e["source"]["ptr"], e["source"]["shape"], e["source"]["stride"], bfloat16, device)
    encoded = FakeTensor(e["out"]["ptr"], e["out"]["shape"], e["out"]["stride"], uint8, device)
    target = FakeTensor(d["target"]["ptr"], d["target"]["shape"], d["target"]["stride"], bfloat16, device)
    tables = FakeTensor(e["tables_ptr"], (544,), (1,), uint8, device)
    fake_torch = _fake_torch(SimpleNamespace(cuda_stream=e["stream"]), uint8=uint8, bfloat16=bfloat16)
    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = FakeLib()
    try:
        with patch.dict(sys.modules, {"torch": fake_torch}), patch.object(
                splitzip_cuda, "_top16_tables", return_value=tables):
            encoded_bytes = splitzip_cuda.encode_top16(source, encoded, e["layer"])
            copied = splitzip_cuda.decode_top16(encoded, target, d["block_ids"], d["raw_bytes"], e["layer"])
    finally:
        splitzip_cuda._LIB = old
    assert (encoded_bytes, copied) == (13, 16)
    assert encode_calls == [tuple(e["expected_call"])]
    assert decode_calls == [tuple(d["expected_call"])]


def test_decode_fixed6_passes_contiguous_native_layout(abi):
    calls = []

    class FakeLib:
        def kvq_splitzip_bf16_decode_fixed6(self, *args):
            calls.append(args)
            return 16

    device = SimpleNamespace(type="cuda")
    uint8, bfloat16 = object(), object()
    f = abi["decode_fixed6"]
    source = FakeTensor(f["source"]["ptr"], f["source"]["shape"], f["source"]["stride"], uint8, device)
    target = FakeTensor(f["target"]["ptr"], f["target"]["shape"], f["target"]["stride"], bfloat16, device)
    fake_torch = _fake_torch(SimpleNamespace(cuda_stream=99), uint8=uint8, bfloat16=bfloat16)
    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = FakeLib()
    try:
        with patch.dict(sys.modules, {"torch": fake_torch}):
            copied = splitzip_cuda.decode_fixed6(source, target, f["block_ids"], f["raw_bytes"])
    finally:
        splitzip_cuda._LIB = old
    assert copied == 16
    assert calls == [tuple(f["expected_call"])]


def test_native_decoders_pass_noncontiguous_block_map(abi):
    fixed_calls, top16_calls = [], []

    class FakeLib:
        def kvq_splitzip_bf16_decode_fixed6(self, *_args):
            raise AssertionError("contiguous decoder used")

        def kvq_splitzip_bf16_decode_fixed6_blocks(self, *args):
            fixed_calls.append(args)
            return 16

        def kvq_splitzip_bf16_decode_top16(self, *_args):
            raise AssertionError("contiguous decoder used")

        def kvq_splitzip_bf16_decode_top16_blocks(self, *args):
            top16_calls.append(args)
            return 16

    device = SimpleNamespace(type="cuda")
    uint8, bfloat16, int64 = object(), object(), object()
    nc = abi["noncontiguous"]

    class FakeBlockIds(FakeTensor):
        def __init__(self):
            super().__init__(nc["block_map_ptr"], (2,), (1,), int64, device)
            self.streams = []

        def record_stream(self, stream):
            self.streams.append(stream)

        def to(self, *_args, **_kwargs):  # the pinned host array's asynchronous upload
            return self

    source = FakeTensor(11, (79,), (1,), uint8, device)
    target = FakeTensor(22, (2, 8, 2), (16, 2, 1), bfloat16, device)
    tables = FakeTensor(44, (544,), (1,), uint8, device)
    block_map = FakeBlockIds()
    current = SimpleNamespace(cuda_stream=99)
    fake_torch = _fake_torch(current, uint8=uint8, bfloat16=bfloat16, int64=int64,
                             tensor=lambda *_a, **_k: block_map)
    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = FakeLib()
    try:
        with patch.dict(sys.modules, {"torch": fake_torch}), patch.object(
                splitzip_cuda, "_top16_tables", return_value=tables):
            fixed = splitzip_cuda.decode_fixed6(source, target, nc["block_ids"], 16)
            top16 = splitzip_cuda.decode_top16(source, target, nc["block_ids"], 16, 7)
    finally:
        splitzip_cuda._LIB = old
    assert (fixed, top16) == (16, 16)
    assert fixed_calls == [tuple(nc["expected_fixed6_blocks_call"])]
    assert top16_calls == [tuple(nc["expected_top16_blocks_call"])]
    assert block_map.streams == [current, current]


@pytest.mark.parametrize("declined", [False, True])
def test_noncontiguous_decode_passes_the_host_table_first(declined):
    """A non-contiguous table of at most HOST_TABLE_BLOCKS ids goes to the host-table
    entry points (no device copy); when they decline (0) the ids are uploaded and
    the device-table entry points run, as without them."""
    host_calls, device_calls = [], []

    def host_entry(*args):
        table = (ctypes.c_longlong * args[4]).from_address(args[8])
        host_calls.append((args[:8], list(table), args[9:]))
        return 0 if declined else 16

    class FakeLib:
        kvq_splitzip_bf16_decode_fixed6 = kvq_splitzip_bf16_decode_top16 = staticmethod(
            lambda *a: pytest.fail("contiguous decoder used"))
        kvq_splitzip_bf16_decode_fixed6_host_blocks = staticmethod(host_entry)
        kvq_splitzip_bf16_decode_top16_host_blocks = staticmethod(host_entry)
        kvq_splitzip_bf16_decode_fixed6_blocks = kvq_splitzip_bf16_decode_top16_blocks = \
            staticmethod(lambda *a: device_calls.append(a) or 16)

    class Uploaded(FakeTensor):
        def __init__(self):
            super().__init__(777, (2,), (1,), object(), SimpleNamespace(type="cuda"))

        def record_stream(self, _stream):
            pass

        def to(self, *_a, **_k):
            return self

    device = SimpleNamespace(type="cuda")
    uint8, bfloat16 = object(), object()
    source = FakeTensor(11, (79,), (1,), uint8, device)
    target = FakeTensor(22, (2, 8, 2), (16, 2, 1), bfloat16, device)
    tables = FakeTensor(44, (544,), (1,), uint8, device)
    uploads = []
    fake_torch = _fake_torch(SimpleNamespace(cuda_stream=99), uint8=uint8, bfloat16=bfloat16,
                             int64=object(), tensor=lambda *a, **k: uploads.append(a) or Uploaded())
    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = FakeLib()
    try:
        with patch.dict(sys.modules, {"torch": fake_torch}), patch.object(
                splitzip_cuda, "_top16_tables", return_value=tables):
            assert splitzip_cuda.decode_fixed6(source, target, [5, 2], 16) == 16
            assert splitzip_cuda.decode_top16(source, target, [5, 2], 16, 7) == 16
    finally:
        splitzip_cuda._LIB = old
    common = (11, 79, 22, 8, 2, 2, 16, 2)
    assert host_calls == [(common, [5, 2], (99,)), (common, [5, 2], (44, 99))]
    if declined:
        assert len(uploads) == 2
        assert device_calls == [common + (5, 777, 99), common + (5, 777, 44, 99)]
    else:
        assert uploads == [] and device_calls == []


@pytest.mark.parametrize("block_ids,raw_bytes", [
    ([], 16), ([3, 3], 16), ([3, 8], 16), ([-1, 2], 16), ([3, 4], 15), ([3, 4], 0), ([3, 4, 5], 16)])
def test_decode_layout_rejects_bad_inputs_before_any_call(block_ids, raw_bytes):
    class FakeLib:
        def __getattr__(self, name):
            raise AssertionError(f"{name} reached")

    class Lib:
        kvq_splitzip_bf16_decode_top16 = staticmethod(lambda *a: pytest.fail("called"))

    device = SimpleNamespace(type="cuda")
    uint8, bfloat16 = object(), object()
    source = FakeTensor(11, (79,), (1,), uint8, device)
    target = FakeTensor(22, (2, 8, 2), (16, 2, 1), bfloat16, device)
    fake_torch = _fake_torch(SimpleNamespace(cuda_stream=1), uint8=uint8, bfloat16=bfloat16,
                             int64=object(), tensor=lambda *a, **k: pytest.fail("tensor built"))
    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = Lib()
    try:
        with patch.dict(sys.modules, {"torch": fake_torch}):
            assert splitzip_cuda.decode_top16(source, target, block_ids, raw_bytes, 0) is None
    finally:
        splitzip_cuda._LIB = old


def test_encoders_decline_non_cuda_and_wrong_dtype():
    device = SimpleNamespace(type="cpu")
    uint8, bfloat16 = object(), object()

    class Lib:
        kvq_splitzip_bf16_encode_top16 = staticmethod(lambda *a: pytest.fail("called"))
        kvq_splitzip_bf16_encode = staticmethod(lambda *a: pytest.fail("called"))

    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = Lib()
    try:
        cpu = FakeTensor(1, (8,), (1,), bfloat16, device)
        assert splitzip_cuda.encode_top16(cpu, cpu, 0) is None
        assert splitzip_cuda.encode_bf16(cpu, cpu) is None
        cuda = SimpleNamespace(type="cuda")
        fake_torch = _fake_torch(SimpleNamespace(cuda_stream=1), uint8=uint8, bfloat16=bfloat16)
        with patch.dict(sys.modules, {"torch": fake_torch}):
            wrong = FakeTensor(1, (8,), (1,), uint8, cuda)
            out = FakeTensor(2, (32,), (1,), uint8, cuda)
            assert splitzip_cuda.encode_top16(wrong, out, 0) is None
            src = FakeTensor(1, (8,), (1,), bfloat16, cuda)
            with pytest.raises(ValueError):
                splitzip_cuda.encode_bf16(src, out, bits=7)
    finally:
        splitzip_cuda._LIB = old


def test_launch_failure_raises_with_last_error():
    class Lib:
        def kvq_splitzip_bf16_encode_top16(self, *args):
            return -1

        def kvq_splitzip_last_error(self):
            return b"top16_encode_kernel: invalid device function"

    device = SimpleNamespace(type="cuda")
    uint8, bfloat16 = object(), object()
    fake_torch = _fake_torch(SimpleNamespace(cuda_stream=1), uint8=uint8, bfloat16=bfloat16)
    old = splitzip_cuda._LIB
    splitzip_cuda._LIB = Lib()
    try:
        with patch.dict(sys.modules, {"torch": fake_torch}), patch.object(
                splitzip_cuda, "_top16_tables", return_value=FakeTensor(44, (544,), (1,), uint8, device)):
            with pytest.raises(RuntimeError, match="invalid device function"):
                splitzip_cuda.encode_top16(FakeTensor(1, (64,), (1,), bfloat16, device),
                                           FakeTensor(2, (256,), (1,), uint8, device), 0)
    finally:
        splitzip_cuda._LIB = old


def test_candidate_paths_honour_environment(monkeypatch):
    monkeypatch.setenv("UNCHAIN_KV_SPLITZIP_LIB", "/nowhere/lib.so")
    assert splitzip_cuda._candidate_paths() == ["/nowhere/lib.so"]
    monkeypatch.delenv("UNCHAIN_KV_SPLITZIP_LIB")
    paths = splitzip_cuda._candidate_paths()
    assert paths[0].endswith("unchainkv_amd/lib/libunchain_kv_splitzip_cuda.so")


# ---------------------------------------------------------------------------
# the real library: loads without a GPU and exports what the header declares

def _declared_symbols():
    header = (ROOT / "include" / "unchain_kv_splitzip.h").read_text()
    return sorted(set(re.findall(r"\b(kvq_splitzip_\w+)\s*\(", header)))


def test_header_declares_the_reference_abi():
    names = _declared_symbols()
    for required in ("kvq_splitzip_last_error", "kvq_splitzip_bf16_encode",
                     "kvq_splitzip_bf16_encode_mode", "kvq_splitzip_bf16_decode_fixed6",
                     "kvq_splitzip_bf16_decode_fixed6_blocks", "kvq_splitzip_bf16_encode_top16",
                     "kvq_splitzip_bf16_decode_top16", "kvq_splitzip_bf16_decode_top16_blocks"):
        assert required in names


def test_library_exports_every_declared_symbol():
    from unchainkv_amd import _build

    if not _build.LIB_PATH.exists():
        _build.build_library()
    lib = ctypes.CDLL(str(_build.LIB_PATH))
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    lib.kvq_splitzip_last_error.restype = ctypes.c_char_p
    assert lib.kvq_splitzip_last_error() == b""


def test_library_declines_bad_preconditions_without_launching():
    """Precondition checks run on the host before any launch (no GPU needed)."""
    from unchainkv_amd import _build

    lib = ctypes.CDLL(str(_build.LIB_PATH))
    u = ctypes.c_ulonglong
    enc = lib.kvq_splitzip_bf16_encode_top16
    enc.argtypes = [u] * 6
    enc.restype = ctypes.c_longlong
    assert enc(0, 8, 64, 4096, 16, 0) == 0          # null source
    assert enc(8, 8, 0, 4096, 16, 0) == 0           # empty
    assert enc(8, 8, 21, 4096, 16, 0) == 0          # E >= 2n
    assert enc(8, 8, 1 << 33, 1 << 40, 16, 0) == 0  # above 2^32-1 words
    e = 5 + 1000 + 500 + 25
    assert enc(8, 8, 1000, ((e + 3) & ~3) + 7, 16, 0) == 0  # no room for the scratch
    dec = lib.kvq_splitzip_bf16_decode_top16_blocks
    dec.argtypes = [u] * 12
    dec.restype = ctypes.c_longlong
    assert dec(8, 1530, 8, 1002, 5, 100, 1000, 100, 0, 0, 16, 0) == 0   # 1002 != 2*5*100
    assert dec(8, 1529, 8, 1000, 5, 100, 500, 100, 0, 0, 16, 0) == 0    # wrong encoded size
    fx = lib.kvq_splitzip_bf16_encode_mode
    fx.argtypes = [u] * 5 + [ctypes.c_int]
    fx.restype = ctypes.c_longlong
    assert fx(8, 8, 1000, 1 << 20, 0, 7) == 0
    assert fx(8, 8, 1000, 100, 0, 6) == 0


def test_writeback_declines_bad_layouts_without_launching():
    """The writeback's host checks (vllm_connector.py:3479-3502: one contiguous run
    per request, enough room, no aliasing) decline before any launch."""
    from unchainkv_amd import _build

    lib = ctypes.CDLL(str(_build.LIB_PATH))
    u = ctypes.c_ulonglong
    arr = lambda *v: (u * len(v))(*v)  # noqa: E731
    wb = lib.kvq_splitzip_top16_writeback_paged
    wb.argtypes = [u, ctypes.POINTER(u), ctypes.POINTER(u), u, u, u, u, u, ctypes.POINTER(u),
                   ctypes.POINTER(u), u, u]
    wb.restype = ctypes.c_longlong
    kv, payloads, status = 1 << 40, 1 << 44, 1 << 46
    plane, bw = 64 * 100, 100  # 64 blocks of 100 words per plane
    # a payload longer than its two runs (2 x 2 x 100 bytes for one block)
    assert wb(payloads, arr(0), arr(401), 1, kv, plane, bw, bw, arr(3), arr(1), status, 0) == 0
    # two requests whose runs overlap (blocks 3..4 and 4..5)
    assert wb(payloads, arr(0, 1000), arr(300, 300), 2, kv, plane, bw, bw, arr(3, 4), arr(2, 2),
              status, 0) == 0
    # a run of several blocks needs blocks packed back to back
    assert wb(payloads, arr(0), arr(300), 1, kv, plane, 2 * bw, bw, arr(3), arr(2), status, 0) == 0
    # the payload buffer lies inside a destination run
    assert wb(kv + 2 * 3 * bw, arr(0), arr(300), 1, kv, plane, bw, bw, arr(3), arr(2), status,
              0) == 0
    # empty run, empty payload, null pointers
    assert wb(payloads, arr(0), arr(300), 1, kv, plane, bw, bw, arr(3), arr(0), status, 0) == 0
    assert wb(payloads, arr(0), arr(0), 1, kv, plane, bw, bw, arr(3), arr(2), status, 0) == 0
    assert wb(payloads, arr(0), arr(300), 1, kv, plane, bw, bw, arr(3), arr(2), 0, 0) == 0
    assert wb(payloads, arr(0), arr(300), 0, kv, plane, bw, bw, arr(3), arr(2), status, 0) == 0


def test_contiguous_run_and_runs():
    from unchainkv_amd import splitzip_cuda
    from unchainkv_amd.connector import _contiguous_runs

    assert splitzip_cuda.contiguous_run([4, 5, 6]) == (4, 3)
    assert splitzip_cuda.contiguous_run([9]) == (9, 1)
    assert splitzip_cuda.contiguous_run([4, 6]) is None
    assert splitzip_cuda.contiguous_run([5, 4]) is None
    assert splitzip_cuda.contiguous_run([]) is None
    assert _contiguous_runs([]) == ()
    assert _contiguous_runs([3, 4, 5, 9, 10, 2]) == ((3, 3), (9, 2), (2, 1))


def test_encoders_reject_a_missing_workspace():
    with pytest.raises(ValueError, match="workspace"):
        splitzip_cuda.encode_top16_paged(None, None, None, None)
    with pytest.raises(ValueError, match="workspace"):
        splitzip_cuda.encode_bf16_paged(None, None, None, None, bits=6)
