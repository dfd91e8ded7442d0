"""Pins the CPU oracle (the checker) before anything is checked against it.

Every codec is compared exhaustively with torch's independent float8_e4m3fn / bfloat16 / float16 casts; the
NVFP4 weight quantizer with the reference's hand-made block and error band (tests/stream_tests.cu:1093-1119);
the tiled layout with literal byte positions from the reference's layout description
(src/core/stream_gemm.cu:15-21,39-46,705-738) and round trips; the GEMM with a float64 product.
"""
import numpy as np
import pytest
import torch

import oracle as O


def test_e4m3_decode_all_codes_vs_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = np.array([O.lib.or_e4m3_decode(int(c)) for c in codes], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))  # signed zeros too
    assert O.lib.or_e4m3_decode(0x7E) == 448.0 and O.lib.or_e4m3_decode(0x01) == 2.0 ** -9


def _torch_e4m3_satfinite(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(x).clamp(-448.0, 448.0)
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_encode_vs_torch_rne():
    rng = np.random.default_rng(1)
    # every midpoint and neighbour of the grid, plus random magnitudes over the whole range and past it
    grid = np.array([O.lib.or_e4m3_decode(c) for c in range(0x7F)], np.float64)
    mids = (grid[1:] + grid[:-1]) / 2
    pts = np.concatenate([grid, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9),
                          rng.uniform(0, 500, 20000), np.exp(rng.uniform(-14, 7, 20000)), [0.0, 1e-30, 447.9, 448,
                                                                                             449, 463, 464, 480, 1e6]])
    x = np.concatenate([pts, -pts]).astype(np.float32)
    got = np.array([O.lib.or_e4m3_encode(float(v)) for v in x], np.uint8)
    assert np.array_equal(got, _torch_e4m3_satfinite(x))


def test_bf16_and_f16_vs_torch():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(20000) * 10.0 ** rng.integers(-40, 38, 20000),
                        [0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 6e-8, 3e-5, 3.3895e38, 1e-45]]).astype(np.float32)
    x = x[np.isfinite(x)]
    want_bf = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got_bf = O.f32_to_bf16(x)
    assert np.array_equal(got_bf, want_bf)
    small = x[np.abs(x) < 1e6]
    want_h = torch.from_numpy(small).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    got_h = np.array([O.lib.or_f16_bits(float(v)) for v in small], np.uint16)
    assert np.array_equal(got_h, want_h)
    for h in range(0, 65536, 7):
        want = torch.tensor([h], dtype=torch.int16 if h < 32768 else torch.int32).to(torch.int16).view(
            torch.float16).float().item() if h < 32768 else None
        if want is not None and not np.isnan(want):
            assert O.lib.or_f16_float(h) == want


def test_e2m1_decode_table_literal():
    # src/core/stream_gemm.cu:782 and tests/stream_tests.cu:34
    want = [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]
    got = [O.lib.or_e2m1_decode(c) for c in range(16)]
    assert got == want and np.signbit(got[8])


def test_e2m1_activation_rne_ties_even():
    # halfway points between codes: 0.25->0, 0.75->1.0(code2), 1.25->1.0, 1.75->2.0, 2.5->2.0, 3.5->4.0, 5->4
    pts = {0.25: 0, 0.75: 2, 1.25: 2, 1.75: 4, 2.5: 4, 3.5: 6, 5.0: 6, 7.0: 7, 0.26: 1, 5.01: 7}
    for v, c in pts.items():
        assert O.lib.or_e2m1_encode_rne(v) == c, v
        assert O.lib.or_e2m1_encode_rne(-v) == c | 8
    assert O.lib.or_e2m1_encode_rne(-0.1) == 8  # sign kept on zero


def test_nvfp4_reference_hand_made_block():
    # tests/stream_tests.cu:1093-1107: amax 2688 = 448 * 6 gives global scale 1 and block scale 448 exactly
    row = [2688, 112, 336, 560, 784, 1120, 1568, 2240, 113, -336, -10, 0, -2688, 338, -1568, 448] + [0] * 16
    w = O.f32_to_bf16(np.array(row, np.float32)).reshape(1, 32)
    v, s, g, _ = O.quant_nvfp4(w)
    want = [7, 0, 1, 2, 3, 4, 5, 6, 1, 9, 0, 0, 15, 2, 13, 2]
    assert g == 1.0
    assert list(s[0]) == [0x7E, 0x01]
    got = [(v[0, i // 2] >> (4 * (i & 1))) & 15 for i in range(16)]
    assert got == want
    assert np.all(v[0, 8:] == 0)


def test_nvfp4_gaussian_error_band():
    # tests/stream_tests.cu:1111-1119: relative squared error of N(0, 0.02) in (0.007, 0.011)
    w = O.normal_bf16(33, 0.02, (256, 1024))
    _, _, _, err = O.quant_nvfp4(w)
    assert 0.007 < err < 0.011


def test_nvfp4_quantizer_matches_torch_recipe():
    # bench/quant/drafter_variants.py:94-104 (nvfp4_codes) evaluated with torch ops here (not imported)
    w = O.normal_bf16(7, 0.02, (32, 256))
    v, s, g, _ = O.quant_nvfp4(w)
    wt = torch.from_numpy(w.view(np.int16)).view(torch.bfloat16).float()
    N, K = wt.shape
    gt = (wt.abs().max() / (448.0 * 6.0)).item()
    b = wt.reshape(N, K // 16, 16)
    sc = (b.abs().amax(-1, keepdim=True) / 6.0 / gt).clamp(min=2 ** -9).to(torch.float8_e4m3fn)
    sv = sc.float() * gt
    bounds = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    y = b / sv
    idx = torch.bucketize(y.abs(), bounds, right=False)
    codes = (idx.to(torch.uint8) | (((y < 0) & (idx > 0)).to(torch.uint8) << 3)).reshape(N, K)
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).numpy()
    assert np.float32(g) == np.float32(gt)
    assert np.array_equal(s, sc.view(torch.uint8).reshape(N, K // 16).numpy())
    assert np.array_equal(v, packed)


def test_fp8_per_channel_matches_torch_recipe():
    # bench/quant/drafter_variants.py:77-81 (fake_fp8) with torch ops
    w = O.normal_f32(5, 0.02, (64, 512))
    q, s = O.quant_fp8_per_channel(w)
    wt = torch.from_numpy(w)
    st = (wt.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12)
    qt = (wt / st).to(torch.float8_e4m3fn)
    assert np.array_equal(s, st[:, 0].numpy())
    assert np.array_equal(q, qt.view(torch.uint8).numpy())
    # the row maximum lands exactly on 448
    assert np.all(np.max(q & 0x7F, axis=1) == 0x7E)


def test_fp8_block_quantizers_reconstruct():
    w = O.normal_f32(9, 0.02, (256, 384))
    q, s = O.quant_fp8_block128(w)
    deq = O.dequant_fp8_block128(q, s)
    assert s.shape == (2, 3)
    rel = np.abs(deq - w).max() / np.abs(w).max()
    assert rel < 2 ** -4  # E4M3 keeps 3 mantissa bits
    # each block's largest magnitude maps to code 0x7e (448)
    for nb in range(2):
        for kb in range(3):
            blk = q[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
            assert (blk & 0x7F).max() == 0x7E
    # scales and codes byte for byte against torch: s = amax / 448 per 128 x 128 block, codes = float8_e4m3fn of
    # w / s (FP32 division, clamped to +-448)
    import torch
    wt = torch.from_numpy(w)
    blocks = wt.view(2, 128, 3, 128)
    st = blocks.abs().amax(dim=(1, 3)) / 448.0
    assert np.array_equal(s, st.numpy())
    qt = (blocks / st[:, None, :, None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn).view(torch.uint8).view(256, 384)
    assert np.array_equal(q, qt.numpy())
    x = O.normal_bf16(10, 1.0, (4, 256))
    xq, xs = O.quant_act_fp8_g128(x)
    xf = O.bf16_to_f32(x)
    for m in range(4):
        for kb in range(2):
            assert xs[m, kb] == np.float32(np.abs(xf[m, kb * 128:(kb + 1) * 128]).max()) / np.float32(448)
    zero = np.zeros((1, 128), np.uint16)
    zq, zs = O.quant_act_fp8_g128(zero)
    assert zs[0, 0] == 1.0 and np.all(zq == 0)
    # the codes: torch's E4M3 cast (round to nearest even) of x * (1 / s), each rounded to FP32, clamped to 448
    for m in range(4):
        for kb in range(2):
            r = np.float32(1) / xs[m, kb]
            v = np.clip(xf[m, kb * 128:(kb + 1) * 128] * r, np.float32(-448), np.float32(448)).astype(np.float32)
            want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(xq[m, kb * 128:(kb + 1) * 128], want)


def test_tiled_fp8_literal_positions():
    # piece p = ((h*2+q)*8+g)*4+t of a 2048-byte block holds W[16*tile+g+8h][128*chunk+32t+16q .. +16]
    N, K = 32, 256
    n_idx, k_idx = np.meshgrid(np.arange(N), np.arange(K), indexing="ij")
    w = ((n_idx * 7 + k_idx * 13) % 251).astype(np.uint8)
    t = O.retile_fp8(w)
    assert t.size == N * K
    assert np.array_equal(t[0:16], w[0, 0:16])          # piece 0
    assert np.array_equal(t[16:32], w[0, 32:48])        # piece 1: t=1
    assert np.array_equal(t[64:80], w[1, 0:16])         # piece 4: g=1
    assert np.array_equal(t[512:528], w[0, 16:32])      # piece 32: q=1
    assert np.array_equal(t[1024:1040], w[8, 0:16])     # piece 64: h=1
    assert np.array_equal(t[2048:2064], w[0, 128:144])  # block 1 = (tile 0, chunk 1)
    assert np.array_equal(t[4096:4112], w[16, 0:16])    # block 2 = (tile 1, chunk 0)
    assert np.array_equal(O.untile_fp8(t, N, K), w)


def test_tiled_nvfp4_literal_positions_and_round_trip():
    N, K = 32, 256
    v = (np.arange(N * K // 2) % 253).astype(np.uint8).reshape(N, K // 2)
    s = (np.arange(N * K // 16) % 97 + 0x28).astype(np.uint8).reshape(N, K // 16)
    t = O.retile_nvfp4(v, s)
    assert t.size == N * K // 2 + N * K // 16
    assert np.array_equal(t[0:16], v[0, 0:16])                # slot 0: row 0, values 0..31
    assert np.array_equal(t[16:32], v[0, 16:32])              # slot 1: t=1
    assert np.array_equal(t[64:80], v[1, 0:16])               # slot 4: row 1
    assert np.array_equal(t[1024:1026], s[0, 0:2])            # scales of slot 0
    assert np.array_equal(t[1026:1028], s[0, 2:4])
    assert np.array_equal(t[1152:1168], v[0, 64:80])          # block (tile 0, chunk 1)
    v2, s2 = O.untile_nvfp4(t, N, K)
    assert np.array_equal(v2, v) and np.array_equal(s2, s)


def test_coded_blob_round_trip():
    w = O.normal_bf16(21, 0.02, (32, 512))
    v, s, g, _ = O.quant_nvfp4(w)
    ok, table, code_of = O.scale_code_table(s)
    assert ok
    blob, raw = O.retile_nvfp4_coded(v, s, code_of)
    N, K = 32, 512
    C = K // 128
    blocks = (N // 16) * C
    assert blob.size == blocks * 1120
    plain = O.retile_nvfp4(v, s)
    for blk in range(blocks):
        assert np.array_equal(blob[blk * 1024:(blk + 1) * 1024], plain[blk * 1152:blk * 1152 + 1024])
        assert np.array_equal(raw[blk * 128:(blk + 1) * 128], plain[blk * 1152 + 1024:(blk + 1) * 1152])
        codes = blob[blocks * 1024 + blk * 96: blocks * 1024 + (blk + 1) * 96]
        for L in range(64):
            lo = codes[2 * (L % 32) + (L // 32)]
            hi = (codes[64 + L % 32] >> (4 * (L // 32))) & 15
            f = int(lo) | (int(hi) << 8)
            assert table[f & 63] == raw[blk * 128 + 2 * L]
            assert table[f >> 6] == raw[blk * 128 + 2 * L + 1]
    too_many = np.arange(65, dtype=np.uint8)
    assert not O.scale_code_table(too_many)[0]


def test_dequant_and_gemm_vs_float64():
    M, N, K = 5, 48, 384
    x = O.normal_bf16(1, 1.0, (M, K))
    w = O.normal_f32(2, 0.02, (N, K))
    q, s = O.quant_fp8_per_channel(w)
    wd = O.dequant_fp8_pc(q, s)
    # dequantized values are exactly e4m3 * s in FP32
    e = np.array([O.lib.or_e4m3_decode(c) for c in range(256)], np.float32)
    assert np.array_equal(wd, (e[q] * s[:, None]).astype(np.float32))
    xf = O.bf16_to_f32(x)
    y = O.gemm_f32(xf, wd)
    y64 = xf.astype(np.float64) @ wd.astype(np.float64).T
    assert np.abs(y - y64).max() <= 1e-5 * np.abs(y64).max()
    yb = O.stream_fp8_pc_bf16(x, q, s)
    assert np.array_equal(yb, O.f32_to_bf16(y))
    # a transposed operand or a dropped scale fails this check
    assert np.abs(O.gemm_f32(xf, e[q]) - y64).max() > 1e-2


def test_nvfp4_dequant_matches_reference_product_order():
    w = O.normal_bf16(3, 0.02, (16, 256))
    v, s, g, _ = O.quant_nvfp4(w)
    d = O.dequant_nvfp4(v, s, g)
    e = np.array([O.lib.or_e4m3_decode(c) for c in range(256)], np.float32)
    f4 = np.array([O.lib.or_e2m1_decode(c) for c in range(16)], np.float32)
    codes = np.stack([v & 15, v >> 4], -1).reshape(16, 256)
    sc = (e[s] * np.float32(g)).astype(np.float32)
    want = (f4[codes] * np.repeat(sc, 16, axis=1)).astype(np.float32)
    assert np.array_equal(d, want)


def test_epilogues():
    g = np.array([-3.0, -0.5, 0.0, 0.7, 9.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, -1.5, 0.25], np.float32)
    h = O.bf16_to_f32(O.epi_silu_mul_bf16(g, u))
    want = (g / (1 + np.exp(-g.astype(np.float64)))) * u
    assert np.allclose(h, want, rtol=2 ** -8)
    r = O.f32_to_bf16(np.array([1.0, -2.0, 0.5, 100.0, 0.0], np.float32))
    y = O.bf16_to_f32(O.epi_residual_bf16(g, r))
    assert np.allclose(y, g + O.bf16_to_f32(r), rtol=2 ** -8)


def test_to_half_rows_closed_form():
    x = O.normal_f32(4, 1.0, (4, 256))
    x[1] = 0.0
    x[2, 7] = 3.0e30
    x[3, 255] = np.inf
    xh, xinv = O.to_half_rows(x)
    for m in range(4):
        mx = np.abs(x[m]).max()
        e = int(np.frexp(np.float32(mx))[1]) if (mx > 0 and np.isfinite(mx)) else 0
        assert xinv[m] == np.float32(2.0 ** (e - 15))
        want = torch.from_numpy((x[m] * np.float32(2.0 ** (15 - e))).astype(np.float32)).to(torch.float16)
        assert np.array_equal(xh[m], want.view(torch.int16).numpy().view(np.uint16))


def test_generator_is_portable():
    a = O.normal_f32(0x4C510000, 1.0, 8)
    b = O.normal_f32(0x4C510000, 1.0, 8)
    assert np.array_equal(a, b)
    big = O.normal_f32(123, 1.0, 200000)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01


def test_rmsnorm_half_vs_float64():
    x = O.normal_f32(91, 1.5, (4, 2048))
    w = O.normal_bf16(92, 0.1, (2048,))
    for gemma in (True, False):
        out, xh, xinv = O.rmsnorm_half(x, w, 1e-6, gemma)
        wf = O.bf16_to_f32(w).astype(np.float64)
        ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6) * ((1 + wf) if gemma else wf)
        assert np.max(np.abs(out - ref)) <= 1e-6 * np.abs(ref).max()
        h2, i2 = O.to_half_rows(out)
        assert np.array_equal(xh, h2) and np.array_equal(xinv, i2)


def test_quant_act_fp8_per_tensor_vs_torch():
    import torch
    x = O.normal_f32(93, 4.0, (8, 512))
    x[0, :3] = [1e9, -1e9, 0.0]
    s = 0.0123
    q = O.quant_act_fp8(x, s)
    xb = torch.from_numpy(x).to(torch.bfloat16).float() * (1.0 / np.float32(s))
    ref = xb.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)


# ---------------- prefill activation producers (reference src/core/prefill_gemm.cu:382-459) ----------------
def test_quant_act_nvfp4_known_answers():
    """A block with amax 6 at input_scale 1 has scale E4M3(1.0) = 0x38 and os = 1, so each code is the E2M1
    round-to-nearest-even of the value itself: every midpoint goes to the even code, a small negative value keeps
    its sign (code 8), low nibble first."""
    v = np.array([[6, -6, 3, 0.1, -0.1, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, -5, 0, -0.0, 0.26]], np.float32)
    q, sf = O.quant_act_nvfp4(v, 1.0)
    assert sf[0, 0] == 0x38
    assert list(q[0]) == [0xF7, 0x05, 0x08, 0x22, 0x44, 0x66, 0x0E, 0x18]
    # a zero block: scale 0 and os 0, codes 0 (8 for negative zero)
    z = np.zeros((1, 16), np.float32)
    z[0, 1] = -0.0
    q, sf = O.quant_act_nvfp4(z, 1.0)
    assert sf[0, 0] == 0 and list(q[0]) == [0x80] + [0] * 7
    # saturating scale: g * amax / 6 above 448 gives 0x7e (448) and the largest value's code 7 or less
    big = np.full((1, 16), 1e6, np.float32)
    q, sf = O.quant_act_nvfp4(big, 1.0)
    assert sf[0, 0] == 0x7E and all(b == 0x77 for b in q[0])
    # input_scale divides: x * (1 / input_scale) scaled blocks give the scale of the unscaled block
    x = O.bf16_to_f32(O.normal_bf16(5, 1.0, (4, 64)))
    q1, s1 = O.quant_act_nvfp4(x, 1.0)
    q2, s2 = O.quant_act_nvfp4(x * 4, 4.0)
    assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_quant_act_nvfp4_block_error_band():
    """Each dequantized value e2m1 * (sv / g) is within half an E2M1 step of the value (round to nearest), with
    the scale from the block's largest magnitude: relative error of the block's largest values below 1/6."""
    x = O.bf16_to_f32(O.normal_bf16(9, 1.0, (8, 256))).astype(np.float32)
    q, sf = O.quant_act_nvfp4(x, 0.5)
    g = 1.0 / 0.5
    codes = np.stack([q & 15, q >> 4], axis=-1).reshape(x.shape)
    vals = np.array([O.lib.or_e2m1_decode(int(c)) for c in codes.reshape(-1)], np.float64).reshape(x.shape)
    sv = np.array([O.lib.or_e4m3_decode(int(b)) for b in sf.reshape(-1)], np.float64).reshape(8, 16)
    deq = vals * np.repeat(sv, 16, axis=1) / g
    step = np.repeat(sv, 16, axis=1) / g  # one unit of E2M1 at scale 1 is 0.5 .. 2 wide: bound by the largest step
    assert np.all(np.abs(deq - x) <= 1.0 * step + 1e-12)
    amax = np.abs(x).reshape(8, 16, 16).max(axis=2)
    assert np.all(np.abs(sv * 6 / g - amax) <= amax / 16 + 1e-12)  # the scale itself: E4M3 of amax / 6


def test_rmsnorm_quant_oracle_consistency():
    """rmsnorm_quant = Gemma RMSNorm, then the quantizers on its output (FP8: quant_act_fp8; NVFP4:
    quant_act_nvfp4), byte for byte."""
    x = O.normal_f32(11, 1.0, (3, 1024))
    w = O.normal_bf16(12, 0.1, (1024,))
    out, q8, _ = O.rmsnorm_quant(x, w, 1e-6, False, 0.05)
    assert np.array_equal(q8, O.quant_act_fp8(out, 0.05))
    out4, q4, sf4 = O.rmsnorm_quant(x, w, 1e-6, True, 0.01)
    qq, ss = O.quant_act_nvfp4(out4, 0.01)
    assert np.array_equal(out, out4) and np.array_equal(q4, qq) and np.array_equal(sf4, ss)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
    ref *= 1.0 + O.bf16_to_f32(w).astype(np.float64)
    assert np.max(np.abs(out - ref)) <= 1e-5 * np.max(np.abs(ref))


# ---------------- independent pins of the prefill checker and the fused SwiGLU quantizer ----------------
def _e4m3_table() -> np.ndarray:
    """E4M3 decode from torch's own float8_e4m3fn (an implementation independent of the oracle's)."""
    return torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()


def test_prefill_fp8_rows_vs_float64_block_product():
    """or_prefill_fp8_rows (the block-scaled prefill checker; reference prefill_gemm.cu:269-342 and the check of
    tests/prefill_tests.cu:179-207) against a float64 product written here from the definition: E4M3 decoded by
    torch, the 1x128 activation scales repeated along K and the 128x128 weight scales repeated along N and K with
    np.repeat. Scales span 2^-6 .. 2^6 so that a wrong scale index moves the result far outside the FP32 bound;
    the same check applied to products with a transposed or shifted scale index fails."""
    M, N, K = 40, 384, 512  # 3 x 4 weight blocks, 4 activation groups per row
    rng = np.random.default_rng(77)
    xq = rng.integers(0, 256, (M, K), dtype=np.uint8)
    wq = rng.integers(0, 256, (N, K), dtype=np.uint8)
    xq[(xq & 0x7F) == 0x7F] = 0x10  # no NaN codes
    wq[(wq & 0x7F) == 0x7F] = 0x21
    xs = np.exp2(rng.integers(-6, 7, (M, K // 128))).astype(np.float32) * rng.uniform(0.5, 1, (M, K // 128)).astype(np.float32)
    ws = np.exp2(rng.integers(-6, 7, (N // 128, K // 128))).astype(np.float32) * rng.uniform(0.5, 1, (N // 128, K // 128)).astype(np.float32)
    rows = np.array([0, 3, 17, 39], np.int32)
    got = O.prefill_fp8_rows(xq, xs, rows, wq, ws).astype(np.float64)

    e = _e4m3_table().astype(np.float64)

    def ref(xs_full, ws_full):
        xd = e[xq[rows]] * xs_full[rows]
        wd = e[wq] * ws_full
        return xd @ wd.T, np.abs(xd) @ np.abs(wd).T

    xs_full = np.repeat(xs.astype(np.float64), 128, axis=1)
    ws_full = np.repeat(np.repeat(ws.astype(np.float64), 128, axis=0), 128, axis=1)
    want, mag = ref(xs_full, ws_full)
    # FP32 accumulation of K exactly-rounded products: |err| <= K * 2^-24 * sum |terms| (a loose, safe bound)
    bound = K * 2.0 ** -24 * mag + 1e-30
    assert np.all(np.abs(got - want) <= bound)
    # the check has teeth: a transposed weight-scale grid, or activation scales shifted by one group, fail it
    xs_shift = np.repeat(np.roll(xs, 1, axis=1).astype(np.float64), 128, axis=1)
    # ws[(n % 128) / 128] (always block row 0) and xs[m][k / 64] (clipped to the last group)
    ws_row0 = np.repeat(np.repeat(ws[np.zeros(N // 128, int)].astype(np.float64), 128, axis=0), 128, axis=1)
    xs_k64 = xs.astype(np.float64)[:, np.minimum(np.arange(K) // 64, K // 128 - 1)]
    for bad_x, bad_w in ((xs_shift, ws_full), (xs_full, ws_row0), (xs_k64, ws_full)):
        b, _ = ref(bad_x, bad_w)
        assert not np.all(np.abs(got - b) <= bound)


def _nvfp4_act_numpy(v: np.ndarray, g: float):
    """The NVFP4 activation encoding written from its definition (reference prefill_gemm.cu:382-394): per block of
    16, sc = E4M3_rne(g * amax / 6) (torch's cast, saturated at 448), os = 1 / (sc * (1 / g)) (0 if sc is 0), and
    each code the E2M1 value nearest to v * os with ties to the even code, saturating at 6, sign kept."""
    M, K = v.shape
    b = v.reshape(M, K // 16, 16).astype(np.float32)
    amax = np.abs(b).max(axis=2)
    t = torch.from_numpy((np.float32(g) * (amax * np.float32(1.0 / 6.0))).astype(np.float32))
    sc = t.clamp(max=448.0).to(torch.float8_e4m3fn)
    sv = sc.float().numpy()
    with np.errstate(divide="ignore"):
        os_ = np.where(sv != 0, np.float32(1.0) / (sv * np.float32(1.0 / g)), np.float32(0)).astype(np.float32)
    y = (b * os_[..., None]).astype(np.float32)
    mag = np.abs(y).astype(np.float64)
    grid = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6], np.float64)
    dist = np.abs(mag[..., None] - grid)
    best = dist.min(axis=-1, keepdims=True)
    cand = dist == best
    # among the nearest codes prefer the even one (ties to even)
    even = np.arange(8) % 2 == 0
    code = np.where((cand & even).any(-1), np.argmax(cand & even, axis=-1), np.argmax(cand, axis=-1))
    code = np.where(mag >= 6, 7, code).astype(np.uint8)
    code |= (np.signbit(y).astype(np.uint8) << 3)
    c = code.reshape(M, K)
    q = (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)
    return q, sc.view(torch.uint8).numpy().reshape(M, K // 16)


def test_quant_act_nvfp4_vs_independent_encoder():
    x = O.bf16_to_f32(O.normal_bf16(21, 1.0, (6, 512)))
    x[0, :16] = [6, -6, 3, 0.1, -0.1, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5, -5, 0, -0.0, 0.26]
    for s in (1.0, 0.37):
        q, sf = O.quant_act_nvfp4(x, s)
        qn, sn = _nvfp4_act_numpy(x, 1.0 / s)
        assert np.array_equal(sf, sn)
        assert np.array_equal(q, qn)


def test_silu_mul_quant_nvfp4_pinned():
    """silu_mul_quant_nvfp4(g, u) (reference prefill_gemm.cu:404-420 with SILU, 613-618) is the NVFP4 encoding of
    bf16(silu(g) * u): checked against the independent encoder on silu computed here in float64 and rounded to
    FP32 (values whose FP32 silu differs by an ulp from expf's may round to another BF16: at most a few codes), and
    against known answers: g = 0 gives a zero block (scale byte 0, codes 0); g = 20, u = 1.5 gives silu = 20
    exactly in FP32, so a block of 30s has scale E4M3(5) and every code 7 (6.0)."""
    g = O.normal_f32(31, 2.0, (8, 1024))
    u = O.normal_f32(32, 1.0, (8, 1024))
    q, sf = O.silu_mul_quant_nvfp4(g, u, 0.5)
    g64 = g.astype(np.float64)
    v = ((g64 / (1.0 + np.exp(-g64))).astype(np.float32) * u).astype(np.float32)
    v = O.bf16_to_f32(O.f32_to_bf16(v))
    qn, sn = _nvfp4_act_numpy(v, 2.0)
    assert np.mean(sf != sn) <= 2e-3
    assert np.mean(q != qn) <= 2e-3
    # known answers
    z = np.zeros((1, 16), np.float32)
    q0, s0 = O.silu_mul_quant_nvfp4(z, np.full((1, 16), 3.0, np.float32), 1.0)
    assert s0[0, 0] == 0 and np.all(q0 == 0)
    big = np.full((1, 16), 20.0, np.float32)
    q1, s1 = O.silu_mul_quant_nvfp4(big, np.full((1, 16), 1.5, np.float32), 1.0)
    assert s1[0, 0] == torch.tensor([5.0]).to(torch.float8_e4m3fn).view(torch.uint8).item() == 0x4A
    assert np.all(q1 == 0x77)
    # large negative g: silu(g) * u is a tiny negative value whose block scale is E4M3 of it / 6
    neg = np.full((1, 16), -30.0, np.float32)
    q2, s2 = O.silu_mul_quant_nvfp4(neg, np.ones((1, 16), np.float32), 1.0)
    t = O.bf16_to_f32(O.f32_to_bf16(np.array([-30.0 / (1.0 + np.exp(30.0))], np.float32)))[0]
    assert s2[0, 0] == torch.tensor([abs(t) / 6.0]).to(torch.float8_e4m3fn).view(torch.uint8).item()


def _fp8_band_check(got, v64, input_scale, rel=4e-6):
    """got codes vs the float64 value: exact where the band fixes the code, one of the band's two codes elsewhere."""
    lo, hi = O.fp8_code_band(v64, input_scale, rel)
    fixed = lo == hi
    assert np.array_equal(got[fixed], lo[fixed])
    assert np.all((got[~fixed] == lo[~fixed]) | (got[~fixed] == hi[~fixed]))
    return float(np.mean(~fixed))


def test_gated_rmsnorm_fp8_oracle_pinned():
    """gated_rmsnorm_fp8 (reference prefill_gemm.cu:461-482, 648-653) against the same formula in float64
    (rstd from the exact sum of squares; the oracle's FP32 butterfly sum and libm expf stay within a few FP32 ulps,
    so codes agree exactly wherever that band does not straddle a BF16 rounding boundary), and known answers
    that a dropped / 128, a missing silu, w read as Gemma's 1 + w, or rows mixed up would break."""
    rows = 96
    x = O.normal_f32(41, 1.5, (rows, 128))
    z = O.normal_f32(42, 2.0, (rows, 128))
    w = O.normal_bf16(43, 0.6, (128,))
    eps, sc = 1e-6, 0.02
    q = O.gated_rmsnorm_fp8(x, z, w, eps, sc)
    x64, z64 = x.astype(np.float64), z.astype(np.float64)
    rstd = 1.0 / np.sqrt((x64 ** 2).sum(axis=1, keepdims=True) / 128 + eps)
    v64 = x64 * rstd * O.bf16_to_f32(w).astype(np.float64) * (z64 / (1 + np.exp(-z64)))
    assert _fp8_band_check(q, v64, sc) < 0.01
    # x = 1, eps = 0: rstd = 1 exactly; w = 1, z = 20: silu(20) = 20 in FP32, so v = 20 and q = E4M3(20 / s)
    one = np.ones((1, 128), np.float32)
    q1 = O.gated_rmsnorm_fp8(one, np.full((1, 128), 20.0, np.float32), np.full(128, 0x3F80, np.uint16), 0.0, 1.0)
    assert np.all(q1 == torch.tensor([20.0]).to(torch.float8_e4m3fn).view(torch.uint8).item())
    # x = 2 everywhere: rstd = 1/2, so x * rstd = 1 again (the mean of squares, not the sum)
    q2 = O.gated_rmsnorm_fp8(2 * one, np.full((1, 128), 20.0, np.float32), np.full(128, 0x3F80, np.uint16), 0.0, 1.0)
    assert np.array_equal(q1, q2)
    # z = 0 gives zero codes; w = -1 flips every sign bit
    assert np.all(O.gated_rmsnorm_fp8(x[:2], np.zeros((2, 128), np.float32), w, eps, sc) & 0x7F == 0)
    qn = O.gated_rmsnorm_fp8(x, z, w ^ 0x8000, eps, sc)
    nz = (q & 0x7F) != 0
    assert np.array_equal(qn[nz], q[nz] ^ 0x80)
    # scaling a row by a power of two leaves its codes (eps = 0): each row is normalized on its own
    s = (2.0 ** (np.arange(rows) % 7 - 3)).astype(np.float32).reshape(rows, 1)
    assert np.array_equal(O.gated_rmsnorm_fp8(x * s, z, w, 0.0, sc), O.gated_rmsnorm_fp8(x, z, w, 0.0, sc))
    # saturation: huge w pushes v * (1 / s) past 448 to the largest finite code
    qs = O.gated_rmsnorm_fp8(one, np.full((1, 128), 20.0, np.float32), np.full(128, 0x4780, np.uint16), 0.0, 1.0)
    assert np.all(qs == 0x7E)


def test_sigmoid_mul_fp8_oracle_pinned():
    """sigmoid_mul_fp8 (reference prefill_gemm.cu:484-494, 662-665) against float64 x * sigmoid(gate), and known
    answers: gate = 0 halves x exactly, a large gate keeps x, a very negative gate gives zero."""
    x = O.normal_f32(51, 3.0, (64, 256))
    gt = O.normal_f32(52, 4.0, (64, 256))
    q = O.sigmoid_mul_fp8(x, gt, 0.05)
    v64 = x.astype(np.float64) / (1 + np.exp(-gt.astype(np.float64)))
    assert _fp8_band_check(q, v64, 0.05) < 0.01
    xs = np.array([[1.0, -3.0, 448.0, 0.5]], np.float32)
    assert np.array_equal(O.sigmoid_mul_fp8(xs, np.zeros_like(xs), 1.0), O.quant_act_fp8(xs / 2, 1.0))
    assert np.array_equal(O.sigmoid_mul_fp8(xs, np.full_like(xs, 40.0), 1.0), O.quant_act_fp8(xs, 1.0))
    assert np.all(O.sigmoid_mul_fp8(xs, np.full_like(xs, -200.0), 1.0) & 0x7F == 0)
