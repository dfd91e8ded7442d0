"""The oracle reproduces the committed golden vectors (tests/golden/vectors.json, written by
tests/golden/make_golden.py) bit for bit, including the reference's own known answers."""
import json
import os
import sys

import numpy as np

import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402

GOLD = json.load(open(os.path.join(HERE, "golden", "vectors.json")))


def test_golden_vectors_unchanged():
    now = make_golden.build()
    assert now == GOLD


def test_reference_known_answers_literal():
    g = GOLD["reference_nvfp4_block"]
    w = O.f32_to_bf16(np.array(g["row"], np.float32)).reshape(1, 32)
    v, s, sc2, _ = O.quant_nvfp4(w)
    assert sc2 == g["scale2"] and list(s[0]) == g["scales"]
    assert [(v[0, i // 2] >> (4 * (i & 1))) & 15 for i in range(16)] == g["codes"]
    assert O.lib.or_e4m3_decode(0x7E) == 448.0 and O.lib.or_e4m3_decode(0x01) == 2.0 ** -9


def test_golden_fp8_tiled_bytes_match_layout_formula():
    t = bytes.fromhex(GOLD["stream_fp8_pc"]["tiled"])
    q = np.frombuffer(bytes.fromhex(GOLD["stream_fp8_pc"]["q"]), np.uint8).reshape(16, 256)
    # block (tile 0, chunk 1), piece 37 = ((h*2+q)*8+g)*4+t with t=1, g=1, q=1, h=0: row 1, values 128+48..+16
    off = 2048 + 37 * 16
    assert t[off:off + 16] == q[1, 128 + 48:128 + 64].tobytes()
