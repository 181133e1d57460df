"""The SMXB binary model form against the JSON it came from.

The decoder here is written from the format's layout (magic, version,
payload size, word-wise FNV-1a checksum, tagged values with raw doubles)
independently of the library's reader, and each converted file must decode
to exactly the document Python's json module reads from the source: same key
order, strings, booleans and bit-identical doubles.  Converting back to JSON
must give that document again, and damaged files must be refused.  Sources:
the models written by the reference's own writer (tests/golden/compact_*)
and the random-init tiny model.  GPU-side, tests/test_compact_models_gpu.py
evaluates a binary file against its JSON source.
"""

import gzip
import json
import os
import shutil
import struct

import numpy as np
import pytest

from _compact import GOLDEN

FNV_OFFSET, FNV_PRIME, MASK = 0xcbf29ce484222325, 0x100000001b3, (1 << 64) - 1


def _checksum(payload):
    pad = (-len(payload)) % 8
    words = np.frombuffer(payload + b"\0" * pad, dtype="<u8")
    h = FNV_OFFSET
    for w in words.tolist():
        h = ((h ^ w) * FNV_PRIME) & MASK
    return h


def _decode(data):
    assert data[:4] == b"SMXB"
    version, size, checksum = struct.unpack_from("<IQQ", data, 4)
    assert version == 1 and size == len(data) - 24
    payload = data[24:]
    assert _checksum(payload) == checksum
    pos = 0

    def count():
        nonlocal pos
        (n,) = struct.unpack_from("<Q", payload, pos)
        pos += 8
        return n

    def string():
        nonlocal pos
        n = count()
        s = payload[pos:pos + n].decode()
        pos += n
        return s

    def value():
        nonlocal pos
        tag = payload[pos]
        pos += 1
        if tag in (0, 1, 2):
            return (None, False, True)[tag]
        if tag == 3:
            (v,) = struct.unpack_from("<d", payload, pos)
            pos += 8
            return v
        if tag == 4:
            return string()
        if tag == 5:
            n = count()
            assert n > 0
            v = np.frombuffer(payload, dtype="<f8", count=n, offset=pos).tolist()
            pos += 8 * n
            return v
        if tag == 6:
            return [value() for _ in range(count())]
        if tag == 7:
            out = {}
            for _ in range(count()):
                k = string()
                out[k] = value()
            return out
        raise AssertionError("unknown tag %d" % tag)

    doc = value()
    assert pos == len(payload)
    return doc


def _same(a, b, where="$"):
    """Exact document equality: key order, types (every JSON number is a
    double in the binary form) and bit-identical numbers."""
    if isinstance(a, dict):
        assert isinstance(b, dict) and list(a) == list(b), where
        for k in a:
            _same(a[k], b[k], where + "." + k)
    elif isinstance(a, list):
        assert isinstance(b, list) and len(a) == len(b), where
        for i, (x, y) in enumerate(zip(a, b)):
            _same(x, y, "%s[%d]" % (where, i))
    elif isinstance(a, bool) or a is None or isinstance(a, str):
        assert type(a) is type(b) and a == b, where
    else:
        assert isinstance(b, (int, float)) and not isinstance(b, bool), where
        assert struct.pack("<d", float(a)) == struct.pack("<d", float(b)), where


def _sources(tmp_path, tiny_model_path):
    out = {"tiny": os.fspath(tiny_model_path)}
    for name in ("compact_medium_m0", "compact_c4", "compact_off23_small"):
        p = tmp_path / (name + ".json")
        with gzip.open(os.path.join(GOLDEN, name + ".json.gz"), "rb") as f, open(p, "wb") as g:
            shutil.copyfileobj(f, g)
        out[name] = p
    return out


def test_binary_form_round_trips_the_json(tmp_path, tiny_model_path):
    from symmetrix import model_format
    for name, src in _sources(tmp_path, tiny_model_path).items():
        with open(src) as f:
            doc = json.load(f)
        binary = tmp_path / (name + ".smxb")
        model_format.convert(src, binary)
        assert model_format.is_binary(binary) and not model_format.is_binary(src)
        _same(doc, _decode(binary.read_bytes()), name)
        back = tmp_path / (name + ".back.json")
        model_format.convert(binary, back, "json")
        with open(back) as f:
            _same(doc, json.load(f), name)
        # binary -> binary is byte-stable
        again = tmp_path / (name + ".again.smxb")
        model_format.convert(back, again)
        assert again.read_bytes() == binary.read_bytes()


def test_damaged_binary_files_are_refused(tmp_path, tiny_model_path):
    from symmetrix import model_format
    binary = tmp_path / "tiny.smxb"
    model_format.convert(tiny_model_path, binary)
    data = binary.read_bytes()
    cases = {
        "flipped": data[:100] + bytes([data[100] ^ 1]) + data[101:],
        "truncated": data[:-9],
        "trailing": data + b"\0",
        "version": data[:4] + struct.pack("<I", 2) + data[8:],
    }
    for what, bad in cases.items():
        p = tmp_path / (what + ".smxb")
        p.write_bytes(bad)
        with pytest.raises(ValueError):
            model_format.convert(p, tmp_path / (what + ".json"), "json")
    # an unknown tag under a correct checksum is refused by the reader itself
    payload = bytearray(data[24:])
    payload[0] = 9
    p = tmp_path / "tag.smxb"
    p.write_bytes(data[:16] + struct.pack("<Q", _checksum(bytes(payload))) + bytes(payload))
    with pytest.raises(ValueError, match="unknown tag"):
        model_format.convert(p, tmp_path / "tag.json", "json")


def test_conversion_refuses_what_is_not_a_model(tmp_path, tiny_model_path):
    from symmetrix import model_format
    other = tmp_path / "other.json"
    other.write_text('{"symmetrix_format_version": 3, "x": [1, 2]}')
    with pytest.raises(ValueError, match="format version 4"):
        model_format.convert(other, tmp_path / "o.smxb")
    with pytest.raises(ValueError):
        model_format.convert(tiny_model_path, tmp_path / "t.bin", "msgpack")
    with pytest.raises(ValueError, match="differ"):
        model_format.convert(tiny_model_path, tiny_model_path)
