""".plx container (pack.py:77-104 layout, pack.py:187-247 writer, generate.py:76-136 reader): CPU tests.

The expected bytes below are assembled field by field from the format
description, with every offset worked out by hand, so a writer that drops
the padding, mis-orders a field or changes an integer width fails.
"""

import struct

import numpy as np
import pytest
import torch

from pollux_amd import castor, plx


def test_golden_layout_small_file():
    cfg = {"a": 1}                       # compact JSON b'{"a":1}' = 7 bytes
    state = {"w": torch.tensor([1, 2, 3], dtype=torch.uint8),
             "s": torch.tensor([[1.5, -2.0]], dtype=torch.float16)}
    got = plx.encode_plx(cfg, state)
    fp = castor.codebook_fingerprint()
    exp = bytearray()
    exp += b"POLLUXH2" + bytes([4]) + bytes(7)                 # 0..15
    exp += (7).to_bytes(4, "little") + b'{"a":1}'              # 16..26
    exp += bytes(37)                                           # 27..63: pad to 64
    exp += b"".join(struct.pack("<f", v) for v in fp)          # 64..127
    exp += (2).to_bytes(4, "little")                           # 128..131
    exp += (1).to_bytes(2, "little") + b"w" + bytes([0, 1])    # name, dtype uint8, ndim 1
    exp += (3).to_bytes(4, "little") + (3).to_bytes(8, "little") + bytes([1, 2, 3])
    exp += (1).to_bytes(2, "little") + b"s" + bytes([2, 2])    # dtype float16, ndim 2
    exp += (1).to_bytes(4, "little") + (2).to_bytes(4, "little") + (4).to_bytes(8, "little")
    exp += bytes.fromhex("003e") + bytes.fromhex("00c0")       # fp16 1.5 = 0x3E00, -2.0 = 0xC000 (LE)
    assert got == bytes(exp)


@pytest.mark.parametrize("cfg_len_target", [43, 44, 45, 107])
def test_config_padding_puts_fingerprint_on_a_64_byte_boundary(cfg_len_target):
    # a JSON string value sized so the compact config is exactly cfg_len_target bytes
    cfg = {"k": "x" * (cfg_len_target - len('{"k":""}'))}
    blob = plx.encode_plx(cfg, {})
    n = int.from_bytes(blob[16:20], "little")
    assert n == cfg_len_target
    fp_off = 20 + n + (-(20 + n)) % 64
    assert fp_off % 64 == 0
    assert blob[20 + n : fp_off] == bytes(fp_off - 20 - n)
    assert struct.unpack("<16f", blob[fp_off : fp_off + 64]) == castor.codebook_fingerprint()
    assert int.from_bytes(blob[fp_off + 64 : fp_off + 68], "little") == 0 and len(blob) == fp_off + 68


def test_round_trip_all_dtypes(tmp_path):
    g = torch.Generator().manual_seed(0)
    state = {
        "blocks.0.attn.q.packed_weights": torch.randint(0, 256, (9 * 48,), dtype=torch.uint8, generator=g),
        "blocks.0.attn.q.sigma_rows": torch.rand(96, generator=g).to(torch.float16),
        "tok_emb.weight_int8": torch.randint(-128, 128, (10, 24), dtype=torch.int8, generator=g),
        "ln_f.weight": torch.randn(24, generator=g),
        "scalar": torch.tensor(3.25),
        "bf16_param": torch.randn(4, 6, generator=g).to(torch.bfloat16),   # stored as float32
        "step": torch.tensor([7, 8], dtype=torch.int64),                   # stored as float32
    }
    cfg = {"n_embd": 24, "n_layer": 1, "name": "Pollux-é"}
    path = tmp_path / "m.plx"
    plx.write_plx(path, cfg, state)
    for mm in (False, True):
        p = plx.read_plx(path, mmap_file=mm)
        assert p["format"] == "pollux_packed_v4" and p["config"] == cfg
        assert p["codebook_fingerprint"] == castor.codebook_fingerprint()
        assert list(p["state_dict"]) == list(state)
        for k, v in state.items():
            r = p["state_dict"][k]
            want = v if v.dtype in (torch.uint8, torch.int8, torch.float16, torch.float32) else v.to(torch.float32)
            assert r.dtype == want.dtype and r.shape == want.shape, k
            assert torch.equal(r, want), k
        del p
    loaded = plx.load_plx(path, "cpu")
    assert loaded["state_dict"]["tok_emb.weight_int8"].dtype == torch.int8
    assert torch.equal(loaded["state_dict"]["ln_f.weight"], state["ln_f.weight"])


def test_reader_errors(tmp_path):
    good = plx.encode_plx({"a": 1}, {"w": torch.zeros(4, dtype=torch.uint8)})
    with pytest.raises(ValueError, match="bad magic"):
        plx.decode_plx(b"POLLUXH1" + good[8:])
    with pytest.raises(ValueError, match="version"):
        plx.decode_plx(good[:8] + bytes([3]) + good[9:])
    with pytest.raises(ValueError, match="truncated"):
        plx.decode_plx(good[:-1])
    bad_len = bytearray(good)
    # data_len field of the only tensor: last 4 data bytes are preceded by the u64 length
    struct.pack_into("<Q", bad_len, len(good) - 4 - 8, 5)
    with pytest.raises(ValueError):
        plx.decode_plx(bytes(bad_len))


def test_fingerprint_check():
    p = plx.decode_plx(plx.encode_plx({}, {}))
    plx.check_fingerprint(p)
    q = plx.decode_plx(plx.encode_plx({}, {}, fingerprint=tuple([0.5] * 16)))
    with pytest.raises(ValueError, match="fingerprint mismatch"):
        plx.check_fingerprint(q)
    with pytest.raises(ValueError, match="Unsupported packed format"):
        plx.check_fingerprint({"format": "pollux_packed_v3"})


def test_numpy_view_of_packed_bytes_is_zero_copy(tmp_path):
    w = torch.arange(900, dtype=torch.int64).remainder(256).to(torch.uint8)
    path = tmp_path / "z.plx"
    plx.write_plx(path, {}, {"x.packed_weights": w})
    p = plx.read_plx(path, mmap_file=True)
    t = p["state_dict"]["x.packed_weights"]
    assert torch.equal(t, w)
    base = np.frombuffer(p["_mmap"], dtype=np.uint8).ctypes.data
    assert base <= t.data_ptr() and t.data_ptr() + t.numel() <= base + len(p["_mmap"])  # a view of the map
