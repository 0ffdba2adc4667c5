"""Format layer: hashes, f16, the .sp-model byte layout, loader checks, bridge.

Pins (no reference code at run time):
  * CRC-32 KAT 0xCBF43926 (include/sp/sp_hash.h:30), SHA-256 / XXH64 against
    hashlib / xxhash;
  * sp_f16_to_f32 exhaustively against numpy's IEEE half (all 63488 finite
    patterns), sp_f32_to_f16 RNE against numpy;
  * the reference session fixture (core/session/qwen3_fixture.c:129-256) restated
    byte-for-byte here must hash to the SHA-256 its test prints
    (e41ecc4b...a65bafe, 88640 B) -- a known answer for the whole header / table /
    hash / placement stack; the bytes then load through this library's loader and
    bridge with the fixture's geometry.
"""
import ctypes
import hashlib
import os
import struct

import numpy as np
import pytest
import xxhash

import spkv
from helpers import model_files

FIXTURE_SHA = "e41ecc4b92cfc09464ec5fe739daf8f37162d1bb830aa89c6542a7e66a65bafe"


def test_crc32_kat():
    assert spkv.l1().sp_crc32(b"123456789", 9) == 0xCBF43926


@pytest.mark.parametrize("n", [0, 1, 55, 56, 63, 64, 65, 1000, 12345])
def test_sha256_xxh64(n):
    msg = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    out = (ctypes.c_uint8 * 32)()
    spkv.l1().sp_sha256(msg, n, out)
    assert bytes(out) == hashlib.sha256(msg).digest()
    for seed in (0, 1, 0x9E3779B97F4A7C15):
        assert spkv.l1().sp_xxh64(msg, n, seed) == xxhash.xxh64(msg, seed=seed).intdigest()


def test_f16_exhaustive():
    L = spkv.l1()
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    mine = np.array([L.sp_f16_to_f32(int(x)) for x in h[fin]], np.float32)
    assert np.array_equal(mine.view(np.uint32), ref[fin].view(np.uint32))
    # weight_dtype_test.c:12-19 known values
    assert L.sp_f16_to_f32(0x3C00) == 1.0 and L.sp_f16_to_f32(0xC000) == -2.0 and L.sp_f16_to_f32(0) == 0.0


def test_f32_to_f16_rne():
    L = spkv.l1()
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(4000) * s for s in (1e-8, 1e-5, 3e-3, 1.0, 3e3)]).astype(np.float32)
    mine = np.array([L.sp_f32_to_f16(float(v)) for v in x], np.uint16)
    assert np.array_equal(mine, x.astype(np.float16).view(np.uint16))


# ---------------------------------------------------------------- fixture KAT
def _sha(b):
    return hashlib.sha256(b).digest()


def build_reference_fixture(q_norm_len=None):
    """Byte-for-byte restatement of the reference's qwen3 session fixture
    (Q8 weights, deterministic patterns, default options).  q_norm_len: write
    the q-norm vectors with that many elements instead of head_dim (a
    malformed but otherwise well-formed file)."""
    NL, E, FF, NH, NKV, HD, V, TOKBLOB = 2, 32, 64, 4, 2, 8, 48, 64
    # tokenizer: 128-byte header + blob i & 0xFF; CRC over [0,52) at 52
    th = struct.pack("<IHHIIIIIIIQQ", 0x4B545053, 0, 1, 128, 2, V, 1, 2, 0, 3, 128, TOKBLOB)
    tk = bytearray(th + b"\0" * (128 - len(th)) + bytes(range(TOKBLOB)))
    struct.pack_into("<I", tk, 52, spkv.l1().sp_crc32(bytes(tk[:52]), 52))
    tk = bytes(tk)
    tensors = []

    def add_q8(name, rows, cols, salt):
        r = np.arange(rows)[:, None]; c = np.arange(cols)[None, :]
        data = (((r * 7 + c * 13 + salt) % 251) - 125).astype(np.int8).tobytes()
        tensors.append((name, 10, [cols, rows], 1, data))
        sc = (0.5 + (np.arange(rows) % 7).astype(np.float32) * np.float32(0.05)).astype(np.float32)
        sc = np.float32(0.5) + (np.arange(rows) % 7).astype(np.float32) * np.float32(0.05)
        tensors.append((name + ".scale", 12, [rows], 4, sc.astype(np.float32).tobytes()))

    def add_f32(name, n):
        f = np.float32(0.9) + (np.arange(n) % 5).astype(np.float32) * np.float32(0.02)
        tensors.append((name, 1, [n], 4, f.astype(np.float32).tobytes()))

    add_q8("token_embd.weight", V, E, 1)
    for L in range(NL):
        s = (L + 1) * 17
        add_f32(f"blk.{L}.attn_norm.weight", E)
        add_q8(f"blk.{L}.attn_q.weight", NH * HD, E, s + 1)
        add_q8(f"blk.{L}.attn_k.weight", NKV * HD, E, s + 2)
        add_q8(f"blk.{L}.attn_v.weight", NKV * HD, E, s + 3)
        add_q8(f"blk.{L}.attn_output.weight", E, NH * HD, s + 4)
        add_f32(f"blk.{L}.attn_q_norm.weight", q_norm_len or HD)
        add_f32(f"blk.{L}.attn_k_norm.weight", HD)
        add_f32(f"blk.{L}.ffn_norm.weight", E)
        add_q8(f"blk.{L}.ffn_gate.weight", FF, E, s + 5)
        add_q8(f"blk.{L}.ffn_up.weight", FF, E, s + 6)
        add_q8(f"blk.{L}.ffn_down.weight", E, FF, s + 7)
    add_f32("output_norm.weight", E)
    tensors.sort(key=lambda t: xxhash.xxh64(t[0].encode(), seed=0).intdigest())
    n = len(tensors)
    data_off = (512 + n * 256 + 65535) // 65536 * 65536
    offs, cur = [], 0
    for t in tensors:
        cur = (cur + 63) // 64 * 64
        offs.append(cur); cur += len(t[4])
    file_size = data_off + (cur + 63) // 64 * 64
    buf = bytearray(file_size)
    tag = b"SP-BLAKE3-v0pl\0\0"
    for i, (name, dt, dims, bsz, data) in enumerate(tensors):
        dd = (dims + [0] * 8)[:8]
        e = struct.pack("<80sII8QQQII32sQ40s", name.encode(), dt, len(dims), *dd, offs[i], len(data),
                        bsz, len(data) // bsz, _sha(tag + data), xxhash.xxh64(name.encode(), seed=0).intdigest(), b"")
        buf[512 + i * 256: 512 + (i + 1) * 256] = e
        buf[data_off + offs[i]: data_off + offs[i] + len(data)] = data
    arch = struct.pack("<9If4BIfI", 2, V, E, NL, NH, NKV, HD, 256, 0, 1e6, 0, 0, 1, 1, FF, 1e-6, 0)
    arch = arch + b"\0" * (192 - len(arch))
    hdr = struct.pack("<IHHIIII256s32sIIQQQQQ", 0x444D5053, 0, 1, 512, 2, 192, 256, arch, _sha(tk), V, n,
                      512, data_off, file_size, 1700000000, 0)
    buf[0:len(hdr)] = hdr
    struct.pack_into("<I", buf, 360, spkv.l1().sp_crc32(bytes(buf[:360]), 360))
    return bytes(buf), tk


def test_reference_fixture_known_answer(tmp_path):
    mb, tk = build_reference_fixture()
    assert len(mb) == 88640
    assert hashlib.sha256(mb).hexdigest() == FIXTURE_SHA
    spm, spt = tmp_path / "fx.spm", tmp_path / "fx.spt"
    spm.write_bytes(mb); spt.write_bytes(tk)
    m = spkv.Model(str(spm), str(spt))
    assert spkv.l1().sp_model_tensor_count(m.h) == 39
    s = spkv.Session(m, 256)            # bridge: Q8 weights (served by the loader, not by the HIP path)
    assert spkv.l1().sp_session_qwen3_model(s.h)
    s.close(); m.close()


def test_bridge_rejects_short_norm(tmp_path):
    """A norm tensor shorter than its role's length (head_dim for q_norm) is
    rejected when the session builds the model view, before anything reads
    the owned copy past its end."""
    mb, tk = build_reference_fixture(q_norm_len=6)
    spm, spt = tmp_path / "short.spm", tmp_path / "short.spt"
    spm.write_bytes(mb); spt.write_bytes(tk)
    m = spkv.Model(str(spm), str(spt))                 # the file itself is well formed
    h = ctypes.c_void_p()
    cfg = spkv.SessionConfig(64, 1, 0, 0, 0, 0)
    rc = spkv.l1().sp_session_create(m.h, ctypes.byref(cfg), None, ctypes.byref(h))
    assert rc == -10 and "attn_q_norm" in spkv.last_error()
    m.close()


def test_reference_fixture_live_sha():
    """When the compiled reference is available, its own fixture builder agrees."""
    import orc
    R = orc.ref_lib()
    if R is None:
        pytest.skip("oracle/_ref not built")
    out = (ctypes.c_uint8 * 32)(); ln = ctypes.c_size_t()
    assert R.refh_qwen3_fixture_sha(out, ctypes.byref(ln)) == 0
    assert bytes(out).hex() == FIXTURE_SHA and ln.value == 88640


# ---------------------------------------------------------------- loader negatives
@pytest.mark.parametrize("mutate,code", [
    (lambda b, t: (b"XXXX" + b[4:], t), -10),                     # bad magic -> SP_EBADFORMAT
    (lambda b, t: (b[:4] + b"\x01\x00" + b[6:], t), -10),         # version_major -> SP_EBADFORMAT
    (lambda b, t: (b[:100] + bytes([b[100] ^ 1]) + b[101:], t), -10),   # CRC mismatch
    (lambda b, t: (b, t[:-1] + bytes([t[-1] ^ 1])), -12),         # tokenizer hash -> SP_ETOKENIZER_HASH
    (lambda b, t: (b + b"\0" * 64, t), -10),                      # file_size mismatch
])
def test_loader_rejects(tmp_path, mutate, code):
    mb, tk = build_reference_fixture()
    mb, tk = mutate(mb, tk)
    spm, spt = tmp_path / "bad.spm", tmp_path / "bad.spt"
    spm.write_bytes(mb); spt.write_bytes(tk)
    h = ctypes.c_void_p()
    rc = spkv.l1().sp_model_load(str(spm).encode(), str(spt).encode(), ctypes.byref(h))
    assert rc == code, spkv.last_error()
    assert spkv.last_error()


def test_loader_missing_file(tmp_path):
    h = ctypes.c_void_p()
    assert spkv.l1().sp_model_load(str(tmp_path / "no.spm").encode(), b"x", ctypes.byref(h)) == -6


# ---------------------------------------------------------------- OK_Q4B producer
def test_q4b_quantizer_roundtrip():
    """code*f16(scale) reconstructs each weight within half a step; codes in
    [-7,7]; the block max is hit exactly up to the f16 rounding of max/7."""
    L = spkv.l1()
    rng = np.random.default_rng(5)
    w = (rng.standard_normal(3840) * 0.02).astype(np.float32)
    codes = np.zeros(1920, np.uint8); bs = np.zeros(120, np.uint16)
    L.sp_q4b_quantize_row(spkv.ptr(w), 3840, spkv.ptr(codes), spkv.ptr(bs))
    lo = (codes & 15).astype(np.int8); hi = (codes >> 4).astype(np.int8)
    q = np.empty(3840, np.int8); q[0::2] = lo; q[1::2] = hi
    q = np.where(q >= 8, q - 16, q)
    assert q.min() >= -7 and q.max() <= 7
    step = bs.view(np.float16).astype(np.float32)
    rec = q.astype(np.float32) * np.repeat(step, 32)
    assert np.all(np.abs(rec - w) <= np.repeat(step, 32) * 0.5 + 1e-12)
    amax = np.abs(w.reshape(120, 32)).max(1)
    assert np.array_equal(bs, (amax / np.float32(7)).astype(np.float32).astype(np.float16).view(np.uint16))


def test_synthetic_model_loads(tmpdir_models):
    spm, spt = model_files(tmpdir_models, "gemma3-tiny")
    m = spkv.Model(spm, spt)
    for name in ("token_embd.weight", "token_embd.weight.bscale", "blk.5.post_ffw_norm.weight", "output_norm.weight"):
        assert spkv.l1().sp_model_find_tensor(m.h, name.encode())
    assert not spkv.l1().sp_model_find_tensor(m.h, b"output.weight")      # tied head
    s = spkv.Session(m, 64)
    s.close(); m.close()


def test_synthetic_model_deterministic(tmp_path):
    a = spkv.write_model(str(tmp_path / "a"), arch_id=2, n_layers=1, hidden=64, n_heads=2, n_kv_heads=1,
                         head_dim=64, n_ff=128, vocab=100, threads=1)
    b = spkv.write_model(str(tmp_path / "b"), arch_id=2, n_layers=1, hidden=64, n_heads=2, n_kv_heads=1,
                         head_dim=64, n_ff=128, vocab=100, threads=4)
    assert open(a[0], "rb").read() == open(b[0], "rb").read()
