"""Safetensors / BF16 decoding (src/binary/safetensors.rs:69-110,
src/binary/bf16.rs:13-15) on the CPU, pinned by the reference's own format
fixture (fixtures/formats/mini.safetensors, copied to tests/golden/formats)
with the values its integration test expects (tests/formats.rs:14-45), and by
the closed form of BF16 widening over every 16-bit pattern. The decode is the
library's (svl_tensor_to_f32, the same code the model loaders run)."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

import svl_amd as S

HERE = os.path.dirname(os.path.abspath(__file__))
MINI = os.path.join(HERE, "golden", "formats", "mini.safetensors")


def test_fixture_decodes_like_the_reference():  # tests/formats.rs:14-45
    raw = open(MINI, "rb").read()
    assert hashlib.sha256(raw).hexdigest() == \
        "caca3b030faeb4ded52275d54c2fca0f2ee0d6b1aeeb8ab1819e0785b1f89ca7"
    (n,) = struct.unpack("<Q", raw[:8])
    assert json.loads(raw[8:8 + n])["__metadata__"]["version"] == "1"
    t = S.read_safetensors(MINI)
    assert sorted(t) == ["alpha", "beta", "empty"]
    assert t["alpha"].dtype == "F32" and t["alpha"].shape == (2, 2)
    assert t["alpha"].to_f32().tolist() == [[1.0, 2.0], [3.0, 4.0]]
    assert t["beta"].dtype == "BF16" and t["beta"].shape == (3,)
    assert t["beta"].to_f32().tolist() == [0.5, -1.0, 2.0]
    assert t["empty"].to_f32().size == 0


def test_bf16_widening_is_exact_for_every_pattern():  # bf16.rs:13-15
    bits = np.arange(1 << 16, dtype=np.uint16)
    got = S.RawTensor("BF16", (bits.size,), bits).to_f32()
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_decode_error_kinds():
    with pytest.raises(S.SvlError) as e:
        S.RawTensor("F16", (2,), np.zeros(2, np.uint16)).to_f32()
    assert e.value.kind == "Unsupported"
    big = S.RawTensor("F32", (1 << 16, 1 << 15), np.zeros(1, np.float32))
    with pytest.raises(S.SvlError) as e:   # 2^31 elements, above the 2^30 cap
        S._check(S.lib().svl_tensor_to_f32(*_view(big), 1))
    assert e.value.kind == "LimitExceeded"


@pytest.mark.parametrize("dtype,itemsize", [("F32", 4), ("BF16", 2)])
@pytest.mark.parametrize("extra", [-1, +1, -4, +6])
def test_payload_length_must_match_the_shape(dtype, itemsize, extra):
    """TensorEntry::to_f32 and bf16::decode_bf16 return Corrupt when the byte
    slice is not numel * 4 (F32) or numel * 2 (BF16) long
    (safetensors.rs:79-88, bf16.rs:40-51); nothing past the payload is read."""
    good = np.arange(6).astype(np.float32 if dtype == "F32" else np.uint16)
    raw = np.frombuffer(good.tobytes() + b"\x00" * 8, np.uint8)
    payload = raw[: good.nbytes + extra]
    with pytest.raises(S.SvlError) as e:
        S.RawTensor(dtype, (2, 3), payload).to_f32()
    assert e.value.kind == "Corrupt"
    want = "bytes, expected" if dtype == "F32" else "BF16 length mismatch"
    assert want in str(e.value)
    assert S.RawTensor(dtype, (2, 3), raw[: good.nbytes]).to_f32().shape == (2, 3)
    with pytest.raises(S.SvlError) as e:   # an empty tensor with a non-empty payload
        S.RawTensor(dtype, (0, 3), raw[:itemsize]).to_f32()
    assert e.value.kind == "Corrupt"


def _view(t):
    import ctypes
    v = S._TensorView()
    v.name = b"big"
    v.dtype = 0
    v.ndim = len(t.shape)
    for i, d in enumerate(t.shape):
        v.shape[i] = d
    v.data = t.data.ctypes.data
    out = np.zeros(1, np.float32)
    _view.keep = (v, out)
    return ctypes.byref(v), ctypes.c_void_p(out.ctypes.data)
