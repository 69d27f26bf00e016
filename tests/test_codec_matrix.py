"""The codec harness (the reference's scripts/bench_codec_matrix.py restated on the
drop-in API): run layout, run count, statistics and geometry on the CPU; on the
GPU every mode passes its checks and the payload's CRC32 is the oracle's for the
same fill."""

import json
import statistics
import zlib

import numpy as np
import pytest

from unchainkv_amd import codec_matrix as cm


@pytest.mark.parametrize("blocks,runs,expected", [
    (10, 3, [0, 1, 2, 3, 5, 6, 7, 9, 10, 11]),
    (5, 10, [0, 2, 4, 6, 8]),
    (7, 1, list(range(7))),
    (4, 4, [0, 2, 4, 6]),
])
def test_block_ids_for_runs(blocks, runs, expected):
    ids = cm.block_ids_for_runs(blocks, runs)
    assert ids == expected
    assert len(ids) == blocks and cm.count_runs(ids) == min(blocks, runs)


def test_block_ids_reject_empty_requests():
    for blocks, runs in ((0, 1), (3, 0)):
        with pytest.raises(ValueError):
            cm.block_ids_for_runs(blocks, runs)


def test_count_runs():
    assert cm.count_runs([]) == 0
    assert cm.count_runs([4]) == 1
    assert cm.count_runs([1, 2, 3, 7, 8, 2]) == 3


def test_summary_statistics():
    values = [float(v) for v in range(1, 21)]
    s = cm.summary(values)
    half = 1.96 * statistics.stdev(values) / np.sqrt(20)
    assert s["mean"] == pytest.approx(10.5)
    assert s["mean_ci95_low"] == pytest.approx(10.5 - half)
    assert s["mean_ci95_high"] == pytest.approx(10.5 + half)
    assert s["p50"] == 10.5
    assert s["p95"] == 19.0   # nearest rank: ceil(0.95 * 20) = 19th value
    assert cm.summary([3.0]) == {"mean": 3.0, "mean_ci95_low": 3.0, "mean_ci95_high": 3.0,
                                 "p50": 3.0, "p95": 3.0}


def test_geometry_and_arguments(tmp_path):
    cfg = tmp_path / "config.json"
    cfg.write_text(json.dumps({"num_hidden_layers": 32, "num_attention_heads": 32,
                               "num_key_value_heads": 8, "hidden_size": 4096}))
    assert cm.load_geometry(cfg) == {"layers": 32, "kv_heads": 8, "head_dim": 128}
    cfg.write_text(json.dumps({"num_hidden_layers": 2, "num_attention_heads": 4,
                               "hidden_size": 256, "head_dim": 96}))
    assert cm.load_geometry(cfg) == {"layers": 2, "kv_heads": 4, "head_dim": 96}
    with pytest.raises(ValueError):
        cm.parse_args(["--model-config", str(cfg), "--tokens", "24", "--mode", "raw",
                       "--runs", "1", "--output", str(tmp_path / "o.json")])


def test_fill_words_escape_is_outside_the_codebook():
    from unchainkv_amd import splitzip_cuda

    books = splitzip_cuda._TOP16_CODEBOOKS
    for layer in range(len(books) // 32):
        k, v, esc = cm.fill_words("top16", layer, books)
        book = books[32 * layer:32 * layer + 32]
        assert (k >> 7) == book[0] and (v >> 7) == book[16]
        assert (esc >> 7) not in book and 1 <= esc >> 7 < 255
    assert cm.fill_words("fixed6", 0, books) == (0x7F15, 0x802A, None)
    assert cm.fill_words("raw", 0, books) == (0x3F95, 0xC02A, None)


def expected_payload(mode, layer, blocks, block_words, books):
    """The payload of the harness's fill, from the oracle."""
    import oracle

    k, v, esc = cm.fill_words(mode, layer, books)
    words = np.empty((2, blocks, block_words), np.uint16)
    words[0], words[1] = k, v
    flat = words.reshape(-1)
    if esc is not None:
        flat[::200] = esc
    if mode == "top16":
        return bytes(oracle.top16_encode(flat, oracle.top16_tables(books[32 * layer:32 * layer + 32])))
    if mode == "fixed6":
        return bytes(oracle.fixed6_encode(flat))
    return bytes([6]) + flat.tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("mode,runs", [("top16", 1), ("top16", 3), ("fixed6", 2), ("raw", 4)])
def test_harness_point_on_the_gpu(tmp_path, mode, runs):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from unchainkv_amd import splitzip_cuda

    print("[case] codec matrix", mode, runs, flush=True)
    cfg = tmp_path / "config.json"
    cfg.write_text(json.dumps({"num_hidden_layers": 32, "num_attention_heads": 32,
                               "num_key_value_heads": 8, "hidden_size": 4096}))
    out = tmp_path / "result.json"
    cm.main(["--model-config", str(cfg), "--tokens", "64", "--mode", mode, "--runs", str(runs),
             "--warmup", "2", "--iterations", "5", "--output", str(out)])
    r = json.loads(out.read_text())
    assert r["passed"] and r["final_bitwise_differences"] == 0
    assert r["actual_runs"] == min(runs, 4) and r["blocks"] == 4
    assert len(r["layer_checks"]) == (32 if mode == "top16" else 1)
    layer = 31 if mode == "top16" else 0
    payload = expected_payload(mode, layer, 4, 16 * 8 * 128, splitzip_cuda._TOP16_CODEBOOKS)
    assert r["encoded_bytes"] == len(payload)
    assert r["encoded_crc32"] == zlib.crc32(payload) & 0xFFFFFFFF
    assert set(r["timing_ms"]) == set(cm.STAGES) and len(r["samples_ms"]["total_ms"]) == 5
