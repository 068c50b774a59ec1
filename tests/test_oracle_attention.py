"""The decode-attention oracle (oracle/attention.py) pinned against torch's
scaled_dot_product_attention, closed forms, page placement and the
reference's own bf16 formula (muserve/model/qwen35_layer_v2.py:493-502)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as att


def make_case(rng, lens, Hq=4, Hkv=1, D=256, spare=3):
    lens = np.asarray(lens)
    pages = [-(-int(n) // 16) for n in lens]
    P = sum(pages) + spare
    perm = rng.permutation(P)
    W = max(1, max(pages))
    table = np.zeros((len(lens), W), dtype=np.int32)
    at = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[at:at + n]
        at += n
    k = rng.standard_normal((P, 16, Hkv, D)).astype(np.float32)
    v = rng.standard_normal((P, 16, Hkv, D)).astype(np.float32)
    q = rng.standard_normal((len(lens), Hq, D)).astype(np.float32)
    return q, k, v, lens, table


@pytest.mark.parametrize("Hq,Hkv", [(4, 1), (4, 2), (8, 1), (1, 1)])
def test_matches_sdpa_float64(Hq, Hkv):
    rng = np.random.default_rng(5)
    q, k, v, lens, table = make_case(rng, [1, 17, 300, 40], Hq=Hq, Hkv=Hkv, D=64)
    scale = 64 ** -0.5
    got = att.decode_attention(q, k, v, lens, table, scale)
    for b, n in enumerate(lens):
        K = torch.from_numpy(att.gather_kv(k, table[b], n)).double()  # [n, Hkv, D]
        V = torch.from_numpy(att.gather_kv(v, table[b], n)).double()
        Kx = K.repeat_interleave(Hq // Hkv, dim=1).permute(1, 0, 2)  # [Hq, n, D]
        Vx = V.repeat_interleave(Hq // Hkv, dim=1).permute(1, 0, 2)
        Q = torch.from_numpy(q[b]).double().unsqueeze(1)  # [Hq, 1, D]
        want = F.scaled_dot_product_attention(Q, Kx, Vx, scale=scale)[:, 0]
        np.testing.assert_allclose(got[b], want.numpy(), rtol=1e-12, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(6)
    q, k, v, lens, table = make_case(rng, [1, 50, 50, 50], Hq=4, Hkv=1, D=32)
    # one token: its V row, whatever the scores
    out = att.decode_attention(q, k, v, lens, table, 0.3)
    np.testing.assert_allclose(out[0], np.repeat(v[table[0, 0], 0], 4, axis=0), rtol=1e-12)
    # constant V over a sequence: that row
    vc = v.copy()
    for p in table[1, :4]:
        vc[p] = vc[table[1, 0], 0]
    out = att.decode_attention(q, k, vc, lens, table, 0.3)
    np.testing.assert_allclose(out[1], np.repeat(vc[table[1, 0], 0], 4, axis=0), rtol=1e-12)
    # equal keys: uniform weights, the mean of V
    kc = k.copy()
    for p in table[2, :4]:
        kc[p] = kc[table[2, 0], 0]
    out = att.decode_attention(q, kc, v, lens, table, 0.3)
    mean = att.gather_kv(v, table[2], 50)[:, 0].astype(np.float64).mean(0)
    np.testing.assert_allclose(out[2], np.tile(mean, (4, 1)), rtol=1e-10, atol=1e-12)
    # one dominant key (token 7): its V row
    kd = k.copy()
    p7, r7 = table[3, 0], 7
    kd[p7, r7, 0] = q[3, 0] * 1e3
    out = att.decode_attention(q, kd, v, lens, table, 1.0)
    np.testing.assert_allclose(out[3, 0], v[p7, r7, 0], rtol=1e-9, atol=1e-9)


def test_page_placement_does_not_matter():
    rng = np.random.default_rng(7)
    q, k, v, lens, table = make_case(rng, [33, 70, 5], Hq=4, Hkv=2, D=32, spare=10)
    P = k.shape[0]
    perm = rng.permutation(P)  # page p moves to perm[p]
    k2, v2 = np.empty_like(k), np.empty_like(v)
    k2[perm], v2[perm] = k, v
    a = att.decode_attention(q, k, v, lens, table, 0.2)
    b = att.decode_attention(q, k2, v2, lens, perm[table].astype(np.int32), 0.2)
    np.testing.assert_array_equal(a, b)


def test_zero_length_is_zero():
    rng = np.random.default_rng(8)
    q, k, v, lens, table = make_case(rng, [0, 3], D=16)
    out = att.decode_attention(q, k, v, lens, table, 0.25)
    assert not out[0].any() and out[1].any()


def test_reference_bf16_formula_is_within_bf16_rounding():
    # The reference computes scores, softmax and the weighted sum in bf16; the
    # oracle in float64. They agree to bf16's few-ulp level.
    rng = np.random.default_rng(9)
    q, k, v, lens, table = make_case(rng, [1, 16, 100, 700], Hq=4, Hkv=1, D=256)
    qb, kb, vb = (torch.from_numpy(x).bfloat16() for x in (q, k, v))
    got = att.reference_bf16(qb, kb, vb, lens, table, 256 ** -0.5).double().numpy()
    want = att.decode_attention(qb.float().numpy(), kb.float().numpy(), vb.float().numpy(),
                                lens, table, 256 ** -0.5)
    err = np.abs(got - want)
    assert err.max() < 0.05 and np.median(err) < 0.005, (err.max(), np.median(err))


def test_dequant_exact_against_torch_and_bf16_dequant():
    # every code, scales across 2^-20 .. 2^10: the values torch's e4m3fn decode
    # times the fp32 scale gives (exact in float64), and bf16(value) is what
    # fp8.dequant_rows writes
    from oracle import fp8
    codes = np.tile(np.arange(256, dtype=np.uint8), (31, 1))
    codes[:, 0x7F] = codes[:, 0xFF] = 0  # leave out the NaN codes
    scales = (2.0 ** np.linspace(-20, 10, 31)).astype(np.float32) * np.float32(1.37)
    got = att.dequant_exact(codes, scales)
    t_codes = torch.from_numpy(codes).view(torch.float8_e4m3fn)
    want = t_codes.double() * torch.from_numpy(scales).double()[:, None]
    np.testing.assert_array_equal(got, want.numpy())
    bf = fp8.dequant_rows(torch.from_numpy(codes), torch.from_numpy(scales))
    np.testing.assert_array_equal(torch.from_numpy(got).bfloat16().float().numpy(), bf.float().numpy())
    assert got[3, 0x80] == 0.0 and np.signbit(got[3, 0x80])  # negative zero stays negative


def test_fp8_attention_close_to_bf16_attention():
    # quantising K/V per row (absmax / 448) moves the output by the fp8
    # rounding only: a 3-bit mantissa, relative error 2^-4 per element at most
    rng = np.random.default_rng(8)
    q, k, v, lens, table = make_case(rng, [1, 40, 333], Hq=4, Hkv=1, D=256)
    from oracle import fp8
    kc, ks = fp8.quantize_rows(torch.from_numpy(k))
    vc, vs = fp8.quantize_rows(torch.from_numpy(v))
    kd = att.dequant_exact(kc.numpy(), ks.numpy())
    vd = att.dequant_exact(vc.numpy(), vs.numpy())
    assert np.abs(kd - k).max() <= np.abs(k).max() * 2.0 ** -4
    exact = att.decode_attention(q, k, v, lens, table, 256 ** -0.5)
    quant = att.decode_attention(q, kd, vd, lens, table, 256 ** -0.5)
    # the codes-and-scales form dequantises the same way, sequence by sequence
    np.testing.assert_array_equal(
        att.decode_attention(q, kc.numpy(), vc.numpy(), lens, table, 256 ** -0.5,
                             ks.numpy(), vs.numpy()), quant)
    assert np.abs(quant - exact).max() < 0.1
    assert np.abs(quant - exact).mean() < 0.01


def _sdpa_varlen(q, k, v, cu_q, cu_k, scale, causal):
    """torch's float64 SDPA per sequence, with the causal mask written out
    bottom-right aligned (query t of nq sees keys 0 .. nk - nq + t)."""
    out = torch.zeros(q.shape, dtype=torch.float64)
    Hq, Hkv = q.shape[1], k.shape[1]
    for b in range(len(cu_q) - 1):
        q0, q1, k0, k1 = int(cu_q[b]), int(cu_q[b + 1]), int(cu_k[b]), int(cu_k[b + 1])
        nq, nk = q1 - q0, k1 - k0
        qq = torch.as_tensor(q[q0:q1]).double().permute(1, 0, 2)            # [Hq, nq, D]
        kk = torch.as_tensor(k[k0:k1]).double().repeat_interleave(Hq // Hkv, 1).permute(1, 0, 2)
        vv = torch.as_tensor(v[k0:k1]).double().repeat_interleave(Hq // Hkv, 1).permute(1, 0, 2)
        mask = None
        if causal:
            pos = torch.arange(nq).unsqueeze(1) + (nk - nq)
            mask = torch.arange(nk).unsqueeze(0) <= pos
            live = mask.any(1)
        o = F.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask, scale=scale)
        if causal:
            o[:, ~live] = 0
        out[q0:q1] = o.permute(1, 0, 2)
    return out.numpy()


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_sdpa_float64(causal):
    g = torch.Generator().manual_seed(21)
    lens_q = [1, 5, 16, 33, 70]
    lens_k = [1, 9, 16, 40, 70]   # a cached prefix where nk > nq
    cu_q = np.concatenate([[0], np.cumsum(lens_q)])
    cu_k = np.concatenate([[0], np.cumsum(lens_k)])
    q = torch.randn(int(cu_q[-1]), 4, 32, generator=g).double().numpy()
    k = torch.randn(int(cu_k[-1]), 1, 32, generator=g).double().numpy()
    v = torch.randn(int(cu_k[-1]), 1, 32, generator=g).double().numpy()
    got = att.prefill_attention(q, k, v, cu_q, 0.3, causal, cu_k=cu_k)
    want = _sdpa_varlen(q, k, v, cu_q, cu_k, 0.3, causal)
    assert np.abs(got - want).max() < 1e-12


def test_prefill_closed_forms_and_paged_equals_contiguous():
    g = torch.Generator().manual_seed(22)
    # one key: every query returns its V row; constant V: the output is V
    q = torch.randn(3, 4, 16, generator=g).numpy()
    k = torch.randn(3, 1, 16, generator=g).numpy()
    v = np.tile(torch.randn(1, 1, 16, generator=g).numpy(), (3, 1, 1))
    out = att.prefill_attention(q, k, v, [0, 3], 1.0, True, cu_k=[0, 3])
    assert np.allclose(out, np.broadcast_to(v[:1], out.shape), atol=1e-12)
    out1 = att.prefill_attention(q[:1], k[:1], v[:1], [0, 1], 1.0, True, cu_k=[0, 1])
    assert np.allclose(out1[0], np.broadcast_to(v[0], (4, 16)))
    # more queries than keys: the first queries see nothing
    out2 = att.prefill_attention(q, k[:1], v[:1], [0, 3], 1.0, True, cu_k=[0, 1])
    assert not out2[:2].any() and np.allclose(out2[2], np.broadcast_to(v[0], (4, 16)))
    # the paged form of the same keys gives the same result
    P = 8
    kc = torch.randn(P, 16, 1, 16, generator=g).numpy()
    vc = torch.randn(P, 16, 1, 16, generator=g).numpy()
    table = np.array([[5, 2, 7]], dtype=np.int32)
    n = 40
    kk = kc[table[0]].reshape(-1, 1, 16)[:n]
    vv = vc[table[0]].reshape(-1, 1, 16)[:n]
    qq = torch.randn(12, 4, 16, generator=g).numpy()
    a = att.prefill_attention(qq, kc, vc, [0, 12], 0.25, True, lens_k=[n], page_table=table)
    b = att.prefill_attention(qq, kk, vv, [0, 12], 0.25, True, cu_k=[0, n])
    assert np.array_equal(a, b)
