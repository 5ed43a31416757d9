"""GPU parity of the token-row gather (embed, weights.metal:90-109) against
the C oracle: bit-exact bf16 rows on every format (NaN positions equal),
the feature-row splice for ids at or past the vocabulary, and native BF16
rows copied as bits."""
import numpy as np
import pytest

import oracle as O
import packers as P
from _util import Guarded, say, upload_at_offset

pytestmark = pytest.mark.gpu

ALL_FORMATS = [P.F32, P.F16, P.BF16, P.Q4_0, P.Q4_1, P.Q8_0, P.Q4_K, P.Q5_K, P.Q6_K, O.MXFP4]


def same_bf16_nan_aware(got, want):
    gn = np.isnan(O.bf16_to_f32(got))
    wn = np.isnan(O.bf16_to_f32(want))
    np.testing.assert_array_equal(gn, wn)
    np.testing.assert_array_equal(got[~gn], want[~wn])


@pytest.mark.parametrize("fmt", ALL_FORMATS)
@pytest.mark.parametrize("k", [512, 2816, 4096])
def test_embed_random_bytes_bit_exact(lib, fmt, k):
    """Random bytes reach every code and subnormal/Inf/NaN scale; rows of
    the vocabulary in any order and repeated, two feature rows, and one id
    past them (a NaN row); weights at byte offset 7 and 0."""
    e, b = O.block_layout(fmt)
    say("embed random bytes", fmt, k)
    vocab = 37
    rb = k // e * b
    data = np.random.default_rng(fmt * 7 + k).integers(0, 256, vocab * rb, dtype=np.uint8)
    feats = O.f32_to_bf16(np.random.default_rng(k).normal(size=(2, k)).astype(np.float32))
    ids = np.array([5, 0, vocab - 1, vocab, 5, vocab + 1, vocab + 9, 18, 36, 2], np.uint32)
    want = O.embed(fmt, data, k, vocab, ids, feats)
    for offset in (7, 0):
        _, wptr = upload_at_offset(lib, data, offset)
        out = Guarded(lib, ids.size * k * 2)
        lib.embed(fmt, wptr, k, vocab, lib.DeviceBuffer.from_array(ids), ids.size, out.ptr,
                  features=lib.DeviceBuffer.from_array(feats), feature_rows=2)
        lib.synchronize()
        same_bf16_nan_aware(out.read(np.uint16).reshape(ids.size, k), want)


def test_embed_bf16_bits_and_no_features(lib):
    """Native BF16 rows are copied as stored (a NaN payload a float round
    trip would quieten survives), and without feature rows every id past
    the vocabulary reads as NaN."""
    k, vocab = 96, 4
    rows = O.f32_to_bf16(np.random.default_rng(3).normal(size=(vocab, k)).astype(np.float32))
    rows[2, 7] = 0x7f81
    rows[1, 0] = 0xff80  # -Inf
    ids = np.array([2, 1, 4, 3], np.uint32)
    out = Guarded(lib, ids.size * k * 2)
    lib.embed(P.BF16, lib.DeviceBuffer.from_array(rows), k, vocab, lib.DeviceBuffer.from_array(ids), ids.size,
              out.ptr)
    lib.synchronize()
    got = out.read(np.uint16).reshape(ids.size, k)
    np.testing.assert_array_equal(got[0], rows[2])
    assert got[0, 7] == 0x7f81 and got[1, 0] == 0xff80
    assert (got[2] == 0x7fc0).all()
    np.testing.assert_array_equal(got, O.embed(P.BF16, rows.view(np.uint8), k, vocab, ids))


def test_embed_baseline_lm_table(lib):
    """A Qwen3-8B-width Q6_K table (4096 wide) through the Embedding operand,
    against the oracle on 64 random token ids."""
    from oco_amd import synth
    k, vocab = 4096, 1000
    say("embed q6_k table")
    w = synth.weights(P.Q6_K, vocab, k, seed=12)
    ids = np.random.default_rng(12).integers(0, vocab, 64).astype(np.uint32)
    emb = lib.Embedding(P.Q6_K, lib.DeviceBuffer.from_array(w), k, vocab)
    out = Guarded(lib, ids.size * k * 2)
    emb.embed(lib.DeviceBuffer.from_array(ids), ids.size, out.ptr)
    lib.synchronize()
    np.testing.assert_array_equal(out.read(np.uint16).reshape(ids.size, k), O.embed(P.Q6_K, w, k, vocab, ids))
