"""The library's host weight quantizers (lq_quantize_*; include/ling_gemm.h) on the CPU: byte for byte the oracle's
restatements (pinned themselves in test_oracle.py), the reference's hand-made NVFP4 block and error band
(tests/stream_tests.cu:1093-1119), torch's float8_e4m3fn cast for the E4M3 encoder, and the error paths."""
import numpy as np
import pytest
import torch

import oracle as O

L = pytest.importorskip("ling_gemm")


def test_nvfp4_hand_made_block():
    # tests/stream_tests.cu:1093-1107: amax 2688 = 448 * 6 -> global scale 1, block scale 448 exactly
    row = [2688, 112, 336, 560, 784, 1120, 1568, 2240, 113, -336, -10, 0, -2688, 338, -1568, 448] + [0] * 16
    w = O.f32_to_bf16(np.array(row, np.float32)).reshape(1, 32)
    v, s, g, _ = L.quantize_nvfp4(w)
    assert g == 1.0 and list(s[0]) == [0x7E, 0x01]
    got = [(v[0, i // 2] >> (4 * (i & 1))) & 15 for i in range(16)]
    assert got == [7, 0, 1, 2, 3, 4, 5, 6, 1, 9, 0, 0, 15, 2, 13, 2]
    assert np.all(v[0, 8:] == 0)


@pytest.mark.parametrize("shape", [(256, 1024), (48, 160), (16, 16)])
def test_nvfp4_matches_oracle_and_error_band(shape):
    w = O.normal_bf16(33, 0.02, shape)
    v, s, g, err = L.quantize_nvfp4(w)
    ov, os_, og, oerr = O.quant_nvfp4(w)
    assert np.array_equal(v, ov) and np.array_equal(s, os_) and np.float32(g) == np.float32(og)
    assert abs(err - oerr) <= 1e-9 * max(oerr, 1e-30)
    if shape == (256, 1024):
        assert 0.007 < err < 0.011  # tests/stream_tests.cu:1111-1119
    z = np.zeros(shape, np.uint16)
    v, s, g, err = L.quantize_nvfp4(z)
    assert g == 1.0 and err == 0.0 and np.all(v == 0)


def test_e4m3_encoder_vs_torch():
    """A row whose largest magnitude is 448 has scale 448 / 448 = 1, so its codes are the encoder's output itself:
    every E4M3 value, every midpoint between neighbours (ties to even), and values just off the midpoints."""
    e = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    e = np.unique(e[np.isfinite(e) & (e >= 0)])
    mids = (e[:-1] + e[1:]) / 2
    vals = np.concatenate([e, mids, np.nextafter(mids, 0), np.nextafter(mids, 1e9), [2 ** -12, 2 ** -10, 1e-30]])
    vals = np.concatenate([vals, -vals]).astype(np.float32)
    K = (len(vals) + 1 + 127) // 128 * 128
    row = np.zeros((1, K), np.float32)
    row[0, 0] = 448.0
    row[0, 1:1 + len(vals)] = vals
    q, s = L.quantize_fp8_channel(row)
    assert s[0] == 1.0
    want = torch.from_numpy(row).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, want)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_fp8_quantizers_match_oracle(dtype):
    w = O.normal_f32(5, 0.02, (256, 384))
    w[3] = 0.0  # an all-zero channel: scale 1e-12
    w[128:256, 256:384] = 0.0  # an all-zero block: scale 1
    if dtype == "bf16":
        wi = O.f32_to_bf16(w)
        wf = O.bf16_to_f32(wi)
    elif dtype == "f16":
        wi = w.astype(np.float16)
        wf = wi.astype(np.float32)
    else:
        wi = wf = w
    q, s = L.quantize_fp8_channel(wi)
    oq, os_ = O.quant_fp8_per_channel(wf)
    assert np.array_equal(q, oq) and np.array_equal(s, os_)
    assert s[3] == np.float32(1e-12)
    qb, sb = L.quantize_fp8_block128(wi)
    oqb, osb = O.quant_fp8_block128(wf)
    assert np.array_equal(qb, oqb) and np.array_equal(sb, osb)
    assert sb[1, 2] == 1.0


def test_block128_ragged_edges():
    """N and K not multiples of 128: the last blocks are partial, scales [ceil(N/128)][ceil(K/128)]."""
    w = O.normal_f32(8, 0.02, (144, 200))
    q, s = L.quantize_fp8_block128(w)
    assert s.shape == (2, 2)
    e = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    for nb in range(2):
        for kb in range(2):
            blk = w[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
            assert s[nb, kb] == np.float32(np.abs(blk).max()) / np.float32(448)
            qb = q[nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
            assert (qb & 0x7F).max() == 0x7E
            want = torch.from_numpy(blk / s[nb, kb]).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(qb, want)


def test_quantizer_errors():
    with pytest.raises(L.LingGemmError, match="multiple of 16"):
        L.quantize_nvfp4(np.zeros((4, 24), np.uint16))
    with pytest.raises(L.LingGemmError, match="dtype"):
        L._check(L.lib.lq_quantize_fp8_channel(L._np_ptr(np.zeros(4, np.float32)), 7, 1, 4,
                                               L._np_ptr(np.zeros(4, np.uint8)), L._np_ptr(np.zeros(1, np.float32))))
    with pytest.raises(L.LingGemmError, match="null"):
        L._check(L.lib.lq_quantize_fp8_block128(None, 0, 1, 4, None, None))
