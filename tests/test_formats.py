"""GGUF / f16 / Q8_0 formats (gguf.ts:67-187): the oracle against closed forms."""
import os
import struct
import tempfile

import numpy as np

from gemma_amd import gguf, synth
from oracle import oracle as orc


def test_f16_exhaustive_against_ieee_half():
    # gguf.ts:95-105 restated; every one of the 65536 codes against numpy's
    # IEEE binary16 -> binary32 conversion (exact for all non-NaN codes).
    codes = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # spot values a dropped term would break
    assert orc.lib().gor_f16_to_f32(0x3C00) == 1.0
    assert orc.lib().gor_f16_to_f32(0x0001) == 2.0 ** -24       # smallest subnormal
    assert orc.lib().gor_f16_to_f32(0x03FF) == 1023 * 2.0 ** -24  # largest subnormal
    assert orc.lib().gor_f16_to_f32(0x7BFF) == 65504.0
    assert np.signbit(orc.lib().gor_f16_to_f32(0x8000))
    assert orc.lib().gor_f16_to_f32(0xFC00) == -np.inf


def test_q8_0_dequant_exact():
    rng = np.random.default_rng(1)
    nb = 4096
    q = rng.integers(-128, 128, size=(nb, 32)).astype(np.int8)
    scales = rng.integers(0, 65536, size=nb).astype(np.uint16)
    scales[(scales & 0x7C00) == 0x7C00] = 0x3C00  # no Inf/NaN scales here
    blocks = gguf.q8_0_blocks(scales.view(np.float16), q)
    got = orc.q8_0_dequant(blocks, nb * 32)
    ref = (q.astype(np.float64) * scales.view(np.float16).astype(np.float64)[:, None]).astype(np.float32).reshape(-1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(got, gguf.dequantize_q8_0_np(blocks, nb * 32))


def test_q8_0_partial_last_block():
    # dequantizeQ8_0 stops at `count` inside the last block (gguf.ts:116)
    blocks = gguf.q8_0_blocks(np.array([2.0, 0.5], np.float16), np.arange(64).reshape(2, 32) - 32)
    got = orc.q8_0_dequant(blocks, 40)
    assert got.shape == (40,)
    assert got[0] == -64.0 and got[31] == -2.0 and got[32] == 0.0 and got[39] == 3.5


def test_pack36_layout():
    # packQ8_0ForGPU (gguf.ts:126-149): f32 scale word, then 8 LE words of quants
    q = (np.arange(32) - 16).astype(np.int8)
    blocks = gguf.q8_0_blocks(np.array([0.25], np.float16), q[None, :])
    packed = orc.q8_0_pack36(blocks, 32)
    assert packed.shape == (9,)
    assert packed[:1].view(np.float32)[0] == 0.25
    assert np.array_equal(packed[1:].view(np.int8), q)


def test_quantize_q8_0_properties():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal(32 * 500) * 0.02).astype(np.float32)
    b = gguf.quantize_q8_0(w).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    q = b[:, 2:].view(np.int8)
    assert q.max() <= 127 and q.min() >= -127
    # the largest |w| of each block maps to +-127
    assert np.all(np.abs(q).max(axis=1) == 127)
    deq = gguf.dequantize_q8_0_np(b.reshape(-1), w.size).reshape(-1, 32)
    err = np.abs(deq - w.reshape(-1, 32)).max(axis=1)
    # rounding to the f32 step (0.5 d) plus the f16 rounding of d itself
    # (|q| <= 127 times a relative 2^-11)
    assert np.all(err <= 0.5 * np.abs(d) * (1 + 1e-6) + 127 * np.abs(d) * 2.0 ** -11)


def test_gguf_roundtrip_reference_layout():
    shape = synth.TINY
    t = synth.make_model(shape, seed=3)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "tiny.gguf")
        synth.write_model_gguf(p, shape, tensors=t)
        raw = open(p, "rb").read()
        magic, version, n_t, n_kv = struct.unpack_from("<IIQQ", raw, 0)
        assert magic == 0x46554747 and version == 3 and n_t == len(t)
        f = gguf.GGUFFile(p)
        assert f.kv["gemma3.embedding_length"] == shape.hidden
        assert f.kv["gemma3.block_count"] == shape.layers
        assert f.kv["tokenizer.ggml.tokens"][106] == "<end_of_turn>"
        assert f.data_offset % 32 == 0  # gguf.ts:90-91
        for name, (typ, dims, data) in t.items():
            ti = f.tensor(name)
            assert ti.ggml_type == typ and ti.dims == dims
            assert ti.nbytes == gguf.tensor_nbytes(typ, int(np.prod(dims)))
            assert np.array_equal(np.asarray(f.tensor_bytes(ti)), np.ascontiguousarray(data).view(np.uint8).ravel())


def test_model_byte_counts():
    # per-token Q8_0 bytes of the two model shapes (34 B per 32 weights)
    assert synth.GEMMA3_1B.q8_bytes() == 1_062_236_160
    assert synth.GEMMA3_270M.q8_bytes() == 284_794_880
