"""Checkpoints in the reference's on-disk format (reference src/checkpoint.c:
1-136): the CKTR training state written after fused Adam+EMA steps is parsed
here byte by byte and its payloads are checked against the oracle's Adam
(src/kernels.cu:170-183, src/optimizer.c:54-69) and EMA (src/ema.c:29-35)
recurrences bit for bit; a CKTR file written here in the reference layout
loads into the library's lists; the reference's error codes hold (missing
file, bad magic, short file, count and size mismatch).  The C side is
tests/ckpt.c in _build/libgradcheck.so."""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "_build" / "libgradcheck.so"
SIZES = [5, 64, 1]
CKTR, CKPT = 0x434B5452, 0x434B5054
TOTAL = 4 * sum(SIZES)


@pytest.fixture(scope="module")
def ck(L):
    assert LIB.exists(), f"{LIB} missing: run __graft_entry__.build()"
    lib = C.CDLL(str(LIB))
    fp = C.POINTER(C.c_float)
    lib.nn_ckpt_test_save.argtypes = [C.c_char_p, C.c_int, C.c_int, fp, C.c_int]
    lib.nn_ckpt_test_load.argtypes = [C.c_char_p, fp, C.c_int, C.POINTER(C.c_int)]
    lib.nn_ckpt_test_weights.argtypes = [C.c_char_p]
    lib.nn_ckpt_test_load_mismatch.argtypes = [C.c_char_p, C.c_int, C.c_int]
    for f in (lib.nn_ckpt_test_save, lib.nn_ckpt_test_load, lib.nn_ckpt_test_weights,
              lib.nn_ckpt_test_load_mismatch):
        f.restype = C.c_int
    return lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def parse(path: Path, training: bool):
    """The reference layout: u32 magic, [i32 step, i32 adam_t], then per list
    i32 count, count x i32 sizes, float32 payloads."""
    raw = path.read_bytes()
    magic, = struct.unpack_from("<I", raw, 0)
    off, hdr = 4, {}
    if training:
        hdr["step"], hdr["adam_t"] = struct.unpack_from("<ii", raw, off)
        off += 8
    lists = []
    for _ in range(4 if training else 1):
        count, = struct.unpack_from("<i", raw, off)
        off += 4
        sizes = list(struct.unpack_from(f"<{count}i", raw, off))
        off += 4 * count
        tensors = []
        for n in sizes:
            tensors.append(np.frombuffer(raw, np.float32, n, off).copy())
            off += 4 * n
        lists.append(tensors)
    assert off == len(raw), "trailing bytes"
    return magic, hdr, lists


def expected_state(orc, steps):
    """The oracle's Adam + EMA recurrences from the harness's initial state."""
    f32 = np.float32
    lr, b1, b2, eps, decay = 1e-3, 0.9, 0.999, 1e-8, 0.99
    w1 = float(f32(1.0) - f32(decay))
    # the harness computes p0 and g in float: 0.01f * (float)(i+1) * (float)(k+1)
    ps = [(f32(0.01) * np.arange(1, n + 1, dtype=f32) * f32(k + 1)).astype(f32) for k, n in enumerate(SIZES)]
    gs = [(f32(0.001) * (np.arange(n, dtype=f32) - f32(3)) * f32(k + 1)).astype(f32) for k, n in enumerate(SIZES)]
    ms = [np.zeros(n, f32) for n in SIZES]
    vs = [np.zeros(n, f32) for n in SIZES]
    sh = [p.copy() for p in ps]
    for t in range(1, steps + 1):
        bc1, bc2 = orc.adam_bias_corrections(b1, b2, t)
        for k in range(len(SIZES)):
            ps[k], ms[k], vs[k] = orc.adam_step(ps[k], ms[k], vs[k], gs[k], lr, b1, b2, eps, bc1, bc2)
            sh[k] = orc.weighted_sum(sh[k], ps[k], decay, w1)
    return [ps, sh, ms, vs]


def test_training_checkpoint_layout_and_values(ck, orc, tmp_path):
    print("[case] CKTR save after 3 fused Adam+EMA steps", flush=True)
    path = tmp_path / "state.cktr"
    out = np.zeros(TOTAL, np.float32)
    assert ck.nn_ckpt_test_save(str(path).encode(), 3, 42, _fp(out), TOTAL) == 0
    magic, hdr, lists = parse(path, True)
    assert magic == CKTR and hdr == {"step": 42, "adam_t": 3}
    assert [[t.size for t in lst] for lst in lists] == [SIZES] * 4
    exp = expected_state(orc, 3)
    names = ("params", "ema_shadow", "adam_m", "adam_v")
    for name, got, ref in zip(names, lists, exp):
        for k in range(len(SIZES)):
            assert_bits_equal(got[k], ref[k], f"{name}[{k}]")
    assert_bits_equal(out, np.concatenate([t for lst in lists for t in lst]), "device state vs file")


def test_training_checkpoint_load_of_reference_layout(ck, rng, tmp_path):
    print("[case] CKTR load of a file written in the reference layout", flush=True)
    path = tmp_path / "ref.cktr"
    vals = [[rng.standard_normal(n).astype(np.float32) for n in SIZES] for _ in range(4)]
    blob = struct.pack("<Iii", CKTR, 1234, 567)
    for lst in vals:
        blob += struct.pack(f"<i{len(SIZES)}i", len(SIZES), *SIZES)
        blob += b"".join(t.tobytes() for t in lst)
    path.write_bytes(blob)
    out = np.zeros(TOTAL, np.float32)
    counters = (C.c_int * 2)()
    assert ck.nn_ckpt_test_load(str(path).encode(), _fp(out), TOTAL, counters) == 0
    assert list(counters) == [1234, 567]
    assert_bits_equal(out, np.concatenate([t for lst in vals for t in lst]), "loaded state")


def test_checkpoint_save_load_roundtrip_and_error_codes(ck, tmp_path):
    print("[case] checkpoint error codes", flush=True)
    w = tmp_path / "w.ckpt"
    assert ck.nn_ckpt_test_weights(str(w).encode()) == 0
    magic, _, lists = parse(w, False)
    assert magic == CKPT and [t.size for t in lists[0]] == SIZES
    assert ck.nn_ckpt_test_load_mismatch(str(w).encode(), 5, 1) == -3   # tensor count
    assert ck.nn_ckpt_test_load_mismatch(str(w).encode(), 6, 0) == -4   # tensor size
    out = np.zeros(TOTAL, np.float32)
    counters = (C.c_int * 2)()
    assert ck.nn_ckpt_test_load(str(tmp_path / "missing").encode(), _fp(out), TOTAL, counters) == -1
    assert ck.nn_ckpt_test_load(str(w).encode(), _fp(out), TOTAL, counters) == -2       # CKPT magic, not CKTR
    t = tmp_path / "t.cktr"
    assert ck.nn_ckpt_test_save(str(t).encode(), 1, 1, _fp(out), TOTAL) == 0
    short = tmp_path / "short.cktr"
    short.write_bytes(t.read_bytes()[:-4])
    assert ck.nn_ckpt_test_load(str(short).encode(), _fp(out), TOTAL, counters) == -2   # short file
    # a file that ends inside the size table: the sizes it holds are checked
    # first, in file order (magic, count, then only the first size here)
    cut = tmp_path / "cut.ckpt"
    cut.write_bytes(w.read_bytes()[:12])
    assert ck.nn_ckpt_test_load_mismatch(str(cut).encode(), 6, 0) == -4  # first size differs
    assert ck.nn_ckpt_test_load_mismatch(str(cut).encode(), 5, 0) == -2  # sizes agree, file short


def test_checkpoint_payload_across_staging_chunks(ck, tmp_path):
    """Payloads stream through a 4 Mi-float staging buffer that may span
    tensors: tensors that cross its boundary, an empty tensor and small ones
    round-trip bit for bit."""
    print("[case] checkpoint payloads across staging chunks", flush=True)
    ck.nn_ckpt_test_roundtrip_sizes.argtypes = [C.c_char_p, C.POINTER(C.c_int), C.c_int]
    ck.nn_ckpt_test_roundtrip_sizes.restype = C.c_int
    sizes = [3, (1 << 22) - 1, 2, 0, (1 << 22) + 5, 7]
    arr = (C.c_int * len(sizes))(*sizes)
    path = tmp_path / "big.ckpt"
    assert ck.nn_ckpt_test_roundtrip_sizes(str(path).encode(), arr, len(sizes)) == 0
    assert path.stat().st_size == 4 + 4 + 4 * len(sizes) + 4 * sum(sizes)
