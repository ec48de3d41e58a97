"""The GGUF reader (strata_hip/gguf.py, after strata_mlx/gguf.py:63-132) on files written by the tests' own writer:
metadata of every value type, tensor shapes in numpy order, bytes at their aligned offsets, float tensors and Q6_K
as float32, shard names. CPU only."""

import numpy as np
import pytest

import independent
from gguf_write import write
from strata_hip import gguf as G
from strata_hip import synth


def test_a_file_reads_back(tmp_path, tables):
    rng = np.random.default_rng(1)
    q2 = synth.random_blocks("Q2_0", 6, 256, rng)
    iq3 = synth.random_blocks("IQ3_S", 2 * 4, 512, rng)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f16 = rng.standard_normal((7,)).astype(np.float16)
    bf = np.array([0x3F80, 0xBF00, 0x37FB, 0x4480], dtype="<u2")  # 1, -0.5, about 3e-5, 1024
    q6 = rng.integers(0, 256, (2, 210), dtype=np.uint8)
    q6[:, 208:210] = np.array([0.01, -0.02], "<f2").view(np.uint8).reshape(2, 2)
    meta = {"general.architecture": "qwen4exp", "qwen4exp.block_count": 2, "qwen4exp.expert_used_count": 10,
            "qwen4exp.rope.freq_base": 1e6, "flag": True, "qwen4exp.ple.layers": [0, 3, 5],
            "tokens": ["a", "bc", "déf"]}
    tensors = [("blk.0.q2", (6, 256), "Q2_0", q2), ("blk.0.experts", (2, 4, 512), "IQ3_S", iq3),
               ("f32", (3, 5), "F32", f32.view(np.uint8)), ("f16", (7,), "F16", f16.view(np.uint8)),
               ("bf16", (4,), "BF16", bf.view(np.uint8)), ("q6", (2, 256), "Q6_K", q6)]
    for align in (32, 64):
        path = str(tmp_path / f"m{align}.gguf")
        write(path, meta, tensors, alignment=align)
        g = G.GGUF(path)
        for k, v in meta.items():
            assert g.meta[k] == pytest.approx(v) if isinstance(v, float) else g.meta[k] == v
        assert g.version == 3 and set(g.tensors) == {t[0] for t in tensors}
        for name, shape, kind, raw in tensors:
            t = g[name]
            assert t.shape == shape and t.type == kind
            np.testing.assert_array_equal(t.data, np.asarray(raw, np.uint8).reshape(-1))
            assert (t.offset - g.tensors["blk.0.q2"].offset) % align == 0
        np.testing.assert_array_equal(G.to_float(g["f32"]), f32)
        np.testing.assert_array_equal(G.to_float(g["f16"]), f16.astype(np.float32))
        want_bf = np.array([0x3F800000, 0xBF000000, 0x37FB0000, 0x44800000], np.uint32).view(np.float32)
        np.testing.assert_array_equal(G.to_float(g["bf16"]), want_bf)  # the bits in the top half of a float32
        assert want_bf[0] == 1.0 and want_bf[3] == 1024.0
        np.testing.assert_allclose(G.to_float(g["q6"]).reshape(-1), independent.dequantize(q6, "Q6_K", 210, None),
                                   rtol=1e-7)
        assert g["blk.0.q2"].quantized and not g["f32"].quantized


def test_bad_files_are_refused(tmp_path):
    path = tmp_path / "x.gguf"
    path.write_bytes(b"GGML" + b"\0" * 60)
    with pytest.raises(ValueError):
        G.GGUF(str(path))
    write(str(path), {}, [("t", (2, 100), "Q2_0", np.zeros(2 * 18, np.uint8))])  # rows of 100: not whole blocks
    with pytest.raises(ValueError):
        G.GGUF(str(path))


def test_shards_are_found_by_name(tmp_path):
    for i in (1, 2, 3):
        write(str(tmp_path / f"model-{i:05d}-of-00003.gguf"), {"part": i}, [])
    parts = G.shards(str(tmp_path / "model-00001-of-00003.gguf"))
    assert [p.meta["part"] for p in parts] == [1, 2, 3]
    write(str(tmp_path / "single.gguf"), {"part": 0}, [])
    assert len(G.shards(str(tmp_path / "single.gguf"))) == 1
