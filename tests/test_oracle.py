"""Pins for the CPU oracle (oracle/qk_oracle.c).

Each check uses something other than the oracle's own formula: torch's dtype
conversions, numpy int64 matmul, float64 recomputation, hand-computed known
answers, or invariants the closed form implies.  Runs on CPU only.
"""
import numpy as np
import pytest
import torch

from op_plugin_amd import workloads as W

F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5
TORCH_DT = {F16: torch.float16, BF16: torch.bfloat16}


def _half_bits(vals, code):
    return W.bits(torch.tensor(vals, dtype=torch.float32).to(TORCH_DT[code]))


# ----------------------------------------------------------------------------- conversions

@pytest.mark.parametrize("code", [F16, BF16])
def test_half_to_f32_exhaustive(oracle, code):
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.convert(pats, code, F32)
    ref = W.from_bits(pats, TORCH_DT[code]).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _f32_probe_patterns():
    rng = np.random.default_rng(1)
    rnd = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    # exact bf16 ties (low 16 bits = 0x8000) and f16 ties (low 13 bits = 0x1000) at many exponents
    hi = rng.integers(0, 2**16, size=20_000, dtype=np.uint64).astype(np.uint32)
    ties_bf = (hi << 16) | 0x8000
    base = rng.integers(0, 2**19, size=20_000, dtype=np.uint64).astype(np.uint32) << 13
    ties_h = base | 0x1000
    # f16 subnormal / overflow neighbourhood
    edge = np.concatenate([np.arange(0x33000000, 0x38900000, 0x1000, dtype=np.uint32),
                           np.arange(0x477fe000, 0x47800100, 0x10, dtype=np.uint32)])
    specials = np.array([0, 0x80000000, 0x7f800000, 0xff800000, 0x7fc00000, 0x00000001], np.uint32)
    return np.concatenate([rnd, ties_bf, ties_h, edge, edge | 0x80000000, specials]).view(np.float32)


@pytest.mark.parametrize("code", [F16, BF16])
def test_f32_to_half_matches_torch(oracle, code):
    f = _f32_probe_patterns()
    got = oracle.convert(f, F32, code)
    ref = W.bits(torch.from_numpy(f.copy()).to(TORCH_DT[code]))
    got_f = W.from_bits(got, TORCH_DT[code]).float().numpy()
    nan = np.isnan(f)
    assert np.all(np.isnan(got_f[nan]))
    assert np.array_equal(got[~nan], ref[~nan])


# ----------------------------------------------------------------------------- dynamic quant

@pytest.mark.parametrize("code", [F16, BF16])
def test_dynamic_quant_known_answers(oracle, code):
    # absmax 127 -> scale exactly 1.0 -> y = rint(x): ties go to even
    row1 = [127.0, 0.5, 1.5, 2.5, -2.5, 3.5, 126.5, -126.5, -0.5, 0.0]
    exp1 = [127, 0, 2, 2, -2, 4, 126, -126, 0, 0]
    # absmax 63.5 -> scale 0.5 -> y = rint(2x): 0.25 -> 0.5 -> 0, 0.75 -> 1.5 -> 2
    row2 = [63.5, 0.25, 0.75, -1.25, 10.0, -63.5, 0.0, 1.0, 2.0, 3.0]
    exp2 = [127, 0, 2, -2, 20, -127, 0, 2, 4, 6]
    row3 = [0.0] * 10                      # zero row: scale 0, y 0
    row4 = [0.0] * 9 + [-3.0]              # single nonzero -> -127
    x = _half_bits([row1, row2, row3, row4], code)
    y, s = oracle.dynamic_quant(x, code)
    assert s.tolist() == [1.0, 0.5, 0.0, np.float32(3.0) / np.float32(127.0)]
    assert y.tolist() == [exp1, exp2, [0] * 10, [0] * 9 + [-127]]


@pytest.mark.parametrize("code", [F16, BF16])
def test_dynamic_quant_non_finite_known_answers(oracle, code):
    """The contract for non-finite rows, by hand: NaN elements do not enter the absmax (fmaxf from 0), the
    clamp is fmaxf / fminf, so a NaN quotient gives -128; a row holding an infinity has s = +Inf, its finite
    elements give 0 and its infinite ones Inf / Inf = NaN, so -128; an all-NaN row has s = 0 and y = 0."""
    nan, inf = float("nan"), float("inf")
    rows = [
        [nan, 127.0, -3.5, 0.5, 2.5, nan],       # s = 1: NaN -> -128, ties to even
        [inf, 5.0, -inf, 0.0, -1.0, 3.0],        # s = +Inf
        [nan, nan, 0.0, 0.0, -0.0, nan],         # NaN only: s = 0, y = 0
        [-inf, 0.0, 0.0, 0.0, 0.0, 0.0],         # a lone -Inf
    ]
    y, s = oracle.dynamic_quant(_half_bits(rows, code), code)
    assert s[0] == 1.0 and s[1] == np.inf and s[2] == 0.0 and s[3] == np.inf
    assert y.tolist() == [[-128, 127, -4, 0, 2, -128], [-128, 0, -128, 0, 0, 0], [0] * 6, [-128, 0, 0, 0, 0, 0]]


def test_dynamic_quant_half_max_rows(oracle):
    """Rows at the fp16 limit +-65504 (NPU_HALF_MAX, op_plugin/utils/OpConstants.h:25): s = RN(65504 / 127) and
    the limits map to +-127; the float64 quotient of every other element is within half a step of y."""
    row = [65504.0, -65504.0, 1.0, 257.0, -32752.0, 0.0, 515.0, -516.0]
    x = _half_bits([row, [-65504.0] + [0.0] * 7], F16)
    y, s = oracle.dynamic_quant(x, F16)
    assert s[0] == np.float32(65504.0) / np.float32(127.0) and s[1] == s[0]
    assert y[0, 0] == 127 and y[0, 1] == -127 and y[1, 0] == -127 and (y[1, 1:] == 0).all()
    q = np.array(row) / np.float64(s[0])
    assert np.all(np.abs(y[0] - q) <= 0.5 + 1e-5)


@pytest.mark.parametrize("code", [F16, BF16])
@pytest.mark.parametrize("K", [1, 7, 64, 4096])
def test_dynamic_quant_invariants(oracle, code, K):
    g = torch.Generator().manual_seed(K)
    x = (torch.randn((33, K), generator=g) * torch.logspace(-3, 3, 33).unsqueeze(1)).to(TORCH_DT[code])
    xf = x.float().numpy().astype(np.float64)
    y, s = oracle.dynamic_quant(W.bits(x), code)
    amax = np.abs(xf).max(axis=1)
    assert np.array_equal(s, (amax.astype(np.float32) / np.float32(127.0)))
    nz = amax > 0
    assert np.all(np.abs(y[nz]).max(axis=1) == 127)
    # y is the integer nearest x/s (the float32 quotient may sit within half an
    # ulp of a .5 boundary, hence the tiny slack)
    q = xf / s[:, None].astype(np.float64)
    assert np.all(np.abs(y - q) <= 0.5 + 1e-5)
    assert np.all((np.sign(y) == np.sign(xf)) | (y == 0))


def test_dynamic_quant_vs_torch_library(oracle):
    """Independent implementation: torch float32 division and torch.round (RNE)."""
    c = W.CFG2[2]
    x = W.w8a8_inputs(c)["x"][:, :2048]
    y, s = oracle.dynamic_quant(W.bits(x), F16)
    xf = x.float()
    st = xf.abs().amax(dim=1) / 127.0
    yt = torch.clamp(torch.round(xf / st[:, None]), -128, 127).to(torch.int8)
    assert np.array_equal(s, st.numpy())
    assert np.array_equal(y, yt.numpy())


def test_dynamic_quant_smooth_scales(oracle):
    g = torch.Generator().manual_seed(3)
    x = torch.randn((5, 96), generator=g).to(torch.float16)
    sm = (0.5 + torch.rand(96, generator=g)).float()
    y, s = oracle.dynamic_quant(W.bits(x), F16, sm.numpy())
    xs = x.float() * sm
    st = xs.abs().amax(dim=1) / 127.0
    yt = torch.clamp(torch.round(xs / st[:, None]), -128, 127).to(torch.int8)
    assert np.array_equal(s, st.numpy())
    assert np.array_equal(y, yt.numpy())


# ----------------------------------------------------------------------------- W8A8

@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (17, 40, 130), (64, 96, 512)])
@pytest.mark.parametrize("transposed", [False, True])
def test_w8a8_acc_vs_numpy(oracle, M, N, K, transposed):
    rng = np.random.default_rng(M * 1000 + K)
    a = rng.integers(-128, 128, (M, K), dtype=np.int64).astype(np.int8)
    w = rng.integers(-128, 128, (K, N), dtype=np.int64).astype(np.int8)
    ref = a.astype(np.int64) @ w.astype(np.int64)
    got = oracle.w8a8_acc(a, np.ascontiguousarray(w.T) if transposed else w, transposed)
    assert np.array_equal(got, ref.astype(np.int32))


def test_w8a8_acc_known_answers(oracle):
    K = 300
    ones = np.ones((4, K), np.int8)
    assert np.all(oracle.w8a8_acc(ones, np.ones((K, 6), np.int8)) == K)
    ext = np.full((2, 1024), -128, np.int8)
    assert np.all(oracle.w8a8_acc(ext, np.full((1024, 3), -128, np.int8)) == 1024 * 16384)
    rng = np.random.default_rng(0)
    x = rng.integers(-128, 128, (5, 64)).astype(np.int8)
    assert np.array_equal(oracle.w8a8_acc(x, np.eye(64, dtype=np.int8)), x.astype(np.int32))


def test_quant_matmul_epilogue_vs_float64(oracle):
    rng = np.random.default_rng(7)
    M, N = 16, 64
    acc = rng.integers(-2**28, 2**28, (M, N)).astype(np.int32)
    s = rng.uniform(1e-3, 1e-2, N).astype(np.float32)
    pt = rng.uniform(1e-3, 1e-1, M).astype(np.float32)
    b = torch.from_numpy(rng.normal(0, 0.1, N).astype(np.float32)).to(torch.bfloat16)
    got = oracle.quant_matmul_epilogue(acc, s, pertoken=pt, bias=W.bits(b), bias_dtype=BF16, out_dtype=F32)
    ref = acc.astype(np.float64) * pt[:, None] * s[None, :] + b.float().numpy()[None, :]
    assert np.allclose(got, ref, rtol=3 * 2.0**-24, atol=0)
    got_bf = oracle.quant_matmul_epilogue(acc, s, pertoken=pt, bias=W.bits(b), bias_dtype=BF16, out_dtype=BF16)
    assert np.array_equal(got_bf, W.bits(torch.from_numpy(got).to(torch.bfloat16)))


def test_quant_matmul_int32_bias_and_int8_out(oracle):
    acc = np.array([[100, -100, 7, 2**20]], np.int32)
    bias = np.array([1, 2, 3, 4], np.int32)
    got = oracle.quant_matmul_epilogue(acc, np.array([1.0], np.float32), bias=bias, bias_dtype=I32,
                                       out_dtype=I32)
    assert got.tolist() == [[101, -98, 10, 2**20 + 4]]
    # int8 requant: rint(acc * 0.5 + 0.25) clamped; 10*0.5+0.25=5.25 -> 5; 2^20 -> 127
    got8 = oracle.quant_matmul_epilogue(acc, np.array([0.5], np.float32), offset=np.array([0.25], np.float32),
                                        out_dtype=I8)
    assert got8.tolist() == [[50, -50, 4, 127]]


# ----------------------------------------------------------------------------- int4 + W4A16

def test_int4_pack_known_words(oracle):
    w = np.array([[0, 1, 2, 3, 4, 5, 6, 7], [-8, -7, -6, -5, -4, -3, -2, -1]], np.int8)
    p = oracle.int4_pack(w)
    assert p[0, 0] == 0x76543210
    assert p[1, 0] == np.int32(np.uint32(0xFEDCBA98).view(np.int32))
    assert np.array_equal(oracle.int4_unpack(p), w)


def test_int4_round_trip_all_positions(oracle):
    vals = np.arange(-8, 8, dtype=np.int8)
    w = np.stack([np.roll(vals, i) for i in range(16)]).reshape(16, 16)
    assert np.array_equal(oracle.int4_unpack(oracle.int4_pack(w)), w)
    tw = torch.from_numpy(w.copy())
    assert np.array_equal(W.int4_pack_cpu(tw).numpy(), oracle.int4_pack(w))


def _nz_word_and_nibble_by_hand(k, n, K):
    """Word index and nibble of element (k, n) in the NZ layout, spelled out step by step."""
    S = K // 128
    block, sup = n // 16, k // 128
    chunk, within = (k % 128) // 8, k % 8
    lane = n % 16 + 16 * (chunk % 4)
    word_in_lane = chunk // 4
    nibble = within // 2 if within % 2 == 0 else 4 + within // 2
    return ((block * S + sup) * 64 + lane) * 4 + word_in_lane, nibble


@pytest.mark.parametrize("k,n,word,nibble", [
    (0, 0, 0, 0), (1, 0, 0, 4), (2, 0, 0, 1), (7, 0, 0, 7),      # one 8-k chunk: even k low, odd k high
    (8, 0, 64, 0),                                                # chunk 1 -> lane 16
    (32, 0, 1, 0),                                                # chunk 4 -> word 1 of lane 0
    (2, 3, 12, 1),                                                # column 3 -> lane 3
    (127, 15, 255, 7),                                            # last element of the first 1 KB block
    (128, 0, 256, 0),                                             # next 128 k: next block of the same columns
    (0, 16, 512, 0),                                              # next 16 columns, after all of K (K = 256)
    (200, 37, ((2 * 2 + 1) * 64 + 5 + 16 * 1) * 4 + 2, 0),       # k%128 = 72: chunk 9 -> g 1, word 2
])
def test_w4_nz_known_positions(oracle, k, n, word, nibble):
    """A single nonzero weight lands in exactly one word at the hand-computed position (K=256, N=48)."""
    K, N = 256, 48
    assert _nz_word_and_nibble_by_hand(k, n, K) == (word, nibble)
    w = np.zeros((K, N), dtype=np.int8)
    w[k, n] = -3   # 0xd as a nibble
    nz = oracle.w4_nz_pack(oracle.int4_pack(w)).ravel().view(np.uint32)
    assert np.count_nonzero(nz) == 1
    assert nz[word] == np.uint32(0xD) << np.uint32(4 * nibble)


def test_w4_nz_round_trip_and_operand_property(oracle):
    """NZ is a bijection of the packed words (round trip on random weights), and each NZ word is the MFMA
    operand the kernels assume: after (word >> 4q) & 0x000f000f, the low half is w[k0+2q, n] and the high half
    w[k0+2q+1, n], k0 = 128*s + 8*(4*j + lane//16), n = 16*b + lane%16."""
    g = np.random.default_rng(3)
    K, N = 384, 80
    w = g.integers(-8, 8, size=(K, N), dtype=np.int8)
    nd = oracle.int4_pack(w)
    nz = oracle.w4_nz_pack(nd)
    assert nz.shape == (N // 16, K // 128, 64, 4)
    assert np.array_equal(oracle.w4_nz_unpack(nz), nd)
    u = nz.view(np.uint32)

    def s4(v):
        return ((v.astype(np.int32) + 8) % 16) - 8

    for b in range(N // 16):
        for s in range(K // 128):
            for lane in range(64):
                for j in range(4):
                    k0, n = 128 * s + 8 * (4 * j + lane // 16), 16 * b + lane % 16
                    word = u[b, s, lane, j]
                    for q in range(4):
                        d = (word >> np.uint32(4 * q)) & np.uint32(0x000F000F)
                        assert s4(d & 0xF) == w[k0 + 2 * q, n]
                        assert s4(d >> 16) == w[k0 + 2 * q + 1, n]


@pytest.mark.parametrize("k,n,byte", [
    (0, 0, 0), (15, 0, 15),                 # one lane's 16 consecutive k
    (16, 0, 16 * 16),                       # next 16 k: lane 16
    (63, 15, 63 * 16 + 15),                 # last byte of the first 1 KB block
    (64, 0, 1024),                          # next 64 k: next block of the same columns (K = 192)
    (0, 16, 3 * 1024),                      # next 16 columns after all of K
    (100, 21, ((1 * 3 + 1) * 64 + 5 + 16 * 2) * 16 + 4),   # k%64 = 36: g 2, byte 4
])
def test_w8_nz_known_positions(oracle, k, n, byte):
    K, N = 192, 32
    w = np.zeros((K, N), dtype=np.int8)
    w[k, n] = -77
    nz = oracle.w8_nz_pack(w).ravel()
    assert np.count_nonzero(nz) == 1 and nz[byte] == -77


def test_w8_nz_round_trip_and_operand_property(oracle):
    g = np.random.default_rng(5)
    K, N = 256, 48
    w = g.integers(-128, 128, size=(K, N), dtype=np.int8)
    nz = oracle.w8_nz_pack(w)
    assert nz.shape == (N // 16, K // 64, 64, 16)
    assert np.array_equal(oracle.w8_nz_unpack(nz), w)
    for b in range(N // 16):
        for s in range(K // 64):
            for lane in range(64):
                k0, n = 64 * s + 16 * (lane // 16), 16 * b + lane % 16
                assert np.array_equal(nz[b, s, lane], w[k0:k0 + 16, n])


def test_w4a16_identity_scale_is_plain_matmul(oracle):
    g = torch.Generator().manual_seed(5)
    M, K, N, G = 3, 256, 16, 128
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    w = torch.randint(-8, 8, (K, N), generator=g, dtype=torch.int8)
    one = torch.ones((K // G, N), dtype=torch.float16)
    zero = torch.zeros((K // G, N), dtype=torch.float16)
    got = oracle.weight_quant_bmm(W.bits(x), BF16, W.int4_pack_cpu(w).numpy(), W.bits(one), W.bits(zero),
                                  F16, G)
    ref = torch.matmul(x.double(), w.double()).float().to(torch.bfloat16)
    assert np.array_equal(got, W.bits(ref))


def test_w4a16_hand_example(oracle):
    # x = all ones (1x128), one group; column n: w = n-8 for n<16 repeated, off = 0.5, scale = 2^-3
    K, N = 128, 16
    x = torch.ones((1, K), dtype=torch.bfloat16)
    w = torch.tensor([[n - 8 for n in range(N)]] * K, dtype=torch.int8)
    sc = torch.full((1, N), 0.125, dtype=torch.float16)
    off = torch.full((1, N), 0.5, dtype=torch.float16)
    got = oracle.weight_quant_bmm(W.bits(x), BF16, W.int4_pack_cpu(w).numpy(), W.bits(sc), W.bits(off), F16, 128)
    expect = [K * (n - 8 + 0.5) * 0.125 for n in range(N)]      # 16*(n-7.5), exact in bf16
    assert W.from_bits(got, torch.bfloat16).float().flatten().tolist() == expect


def test_w4a16_linearity(oracle):
    case = W.W4A16Case(M=4, N=64, K=256)
    d = W.w4a16_inputs(case, seed=2)
    a = oracle.weight_quant_bmm(W.bits(d["x"]), BF16, d["w_packed"].numpy(), W.bits(d["scale"]),
                                W.bits(d["offset"]), F16, 128)
    b = oracle.weight_quant_bmm(W.bits(d["x"] * 2), BF16, d["w_packed"].numpy(), W.bits(d["scale"]),
                                W.bits(d["offset"]), F16, 128)
    af = W.from_bits(a, torch.bfloat16).float()
    bf = W.from_bits(b, torch.bfloat16).float()
    assert torch.equal(af * 2, bf)


def test_w4a16_matches_float64_dequant(oracle):
    """Against torch float64: x @ ((w + off) * scale) with scales expanded per group."""
    case = W.W4A16Case(M=5, N=48, K=384)
    d = W.w4a16_inputs(case, seed=4)
    got = oracle.weight_quant_bmm(W.bits(d["x"]), BF16, d["w_packed"].numpy(), W.bits(d["scale"]),
                                  W.bits(d["offset"]), F16, 128)
    wf = (d["w"].double() + d["offset"].double().repeat_interleave(128, 0)) * \
        d["scale"].double().repeat_interleave(128, 0)
    ref = (d["x"].double() @ wf).float().to(torch.bfloat16)
    diff = (W.from_bits(got, torch.bfloat16).float() - ref.float()).abs()
    assert diff.max().item() <= 2.0**-7 * ref.float().abs().max().item()


# ----------------------------------------------------------------------------- MLP neighbours

def test_rms_norm_reference_closed_form(oracle):
    """numpy closed form of test/test_custom_ops/test_npu_rms_norm.py:10-17 (float64 here)."""
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.uniform(0, 100, (8, 256)).astype(np.float32)).to(torch.bfloat16)
    gm = torch.from_numpy(rng.uniform(0, 100, 256).astype(np.float32)).to(torch.bfloat16)
    y, rstd = oracle.rms_norm(W.bits(x), BF16, W.bits(gm))
    xf = x.double().numpy()
    variance = np.mean(np.power(xf, 2), axis=-1, keepdims=True)
    r = 1 / np.sqrt(variance + 1e-6)
    ref = xf * r * gm.double().numpy()
    assert np.allclose(rstd, r, rtol=1e-6)
    assert np.array_equal(y, W.bits(torch.from_numpy(ref).float().to(torch.bfloat16)))


def test_rms_norm_f32_vs_torch_rms_norm(oracle):
    """float32 RMSNorm against torch.nn.functional.rms_norm (a library routine) in float64, on the
    reference's golden distribution (uniform(0, 100) x and gamma) and on signed data; and a row of
    three values worked by hand: x = (3, 4, 0), mean(x^2) = 25/3, rstd = sqrt(3)/5."""
    rng = np.random.default_rng(1)
    for x, gm in [(rng.uniform(0, 100, (6, 384)), rng.uniform(0, 100, 384)),
                  (rng.standard_normal((5, 96)) * 3, 1 + 0.02 * rng.standard_normal(96))]:
        x, gm = x.astype(np.float32), gm.astype(np.float32)
        y, rstd = oracle.rms_norm_f32(x, gm, 1e-6)
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (x.shape[-1],),
                                           torch.from_numpy(gm).double(), eps=1e-6)
        assert np.array_equal(y, ref.float().numpy())
        ms = (torch.from_numpy(x).double() ** 2).mean(-1, keepdim=True)
        assert np.allclose(rstd, (1 / torch.sqrt(ms + 1e-6)).numpy(), rtol=1e-7)
    y, rstd = oracle.rms_norm_f32(np.array([[3.0, 4.0, 0.0]], np.float32), np.array([1.0, 2.0, 5.0], np.float32), 0.0)
    r = np.sqrt(3.0) / 5.0
    assert rstd[0, 0] == np.float32(r)
    assert np.array_equal(y[0], np.array([3 * r, 8 * r, 0.0], np.float32))


def test_swiglu_vs_torch_silu(oracle):
    g = torch.Generator().manual_seed(9)
    h = (3 * torch.randn((4, 64), generator=g)).to(torch.bfloat16)
    got = oracle.swiglu(W.bits(h), BF16)
    a, b = h.double().chunk(2, dim=-1)
    ref = (torch.nn.functional.silu(a) * b).float().to(torch.bfloat16)
    assert np.array_equal(got, W.bits(ref))


# ----------------------------------------------------------------------------- static quantization

_QT = {"qint8": (torch.qint8, 4), "quint8": (torch.quint8, 6), "qint32": (torch.qint32, 5)}


@pytest.mark.parametrize("qname", list(_QT))
def test_quantize_per_tensor_vs_torch(oracle, qname):
    """torch.quantize_per_tensor (CPU, .int_repr()) on random data, planted exact ties and values past the clamp
    bounds.  Quotients beyond the int32 range are left out of the comparison: torch's vectorized CPU path wraps
    them (-5e13 becomes +127 for qint8); the oracle saturates (test_quantize_hand_cases)."""
    dt, code = _QT[qname]
    g = torch.Generator().manual_seed(1)
    for scale, zp in ((0.05, 0), (0.0173, 3), (1.0, 0), (0.5, -7), (3e-3, 101), (2e-5, 1234567)):
        if dt == torch.quint8 and not 0 <= zp <= 255:
            zp = 10
        if dt == torch.qint8 and not -128 <= zp <= 127:
            zp = -5
        x = torch.randn(4096, generator=g) * 4
        j = torch.randint(-300, 300, (512,), generator=g).float()
        x[:512] = (j + 0.5) * scale                       # exact ties after the multiply by 1/scale
        x[512:518] = torch.tensor([1e6, -1e6, 0.0, -0.0, 200.0, -200.0])
        keep = (x.double() / scale).abs() < 2.0**31
        t = torch.quantize_per_tensor(x, scale, zp, dt).int_repr().numpy()
        r = oracle.quantize(x.numpy(), oracle.F32, np.array([scale]), np.array([zp]), None, code)
        assert np.array_equal(t[keep.numpy()].astype(np.int64), r[keep.numpy()].astype(np.int64))


@pytest.mark.parametrize("qname", list(_QT))
@pytest.mark.parametrize("axis", [0, 1, 2, -1])
def test_quantize_per_channel_vs_torch(oracle, qname, axis):
    dt, code = _QT[qname]
    g = torch.Generator().manual_seed(2)
    x = torch.randn(6, 40, 7, generator=g) * 3
    C = x.shape[axis]
    sc = torch.rand(C, generator=g, dtype=torch.float64) * 0.1 + 1e-3
    lo = 0 if dt == torch.quint8 else -20
    zp = torch.randint(lo, 20, (C,), generator=g, dtype=torch.int64)
    # the reference wraps a negative axis (op_plugin/ops/base_ops/aclops/QuantizePerChannelKernelNpu.cpp:75); torch
    # takes only the wrapped one
    t = torch.quantize_per_channel(x, sc, zp, axis % x.dim(), dt).int_repr().numpy()
    r = oracle.quantize(x.numpy(), oracle.F32, sc.float().numpy(), zp.numpy(), axis, code)
    assert np.array_equal(t.astype(np.int64), r.astype(np.int64))


def test_quantize_hand_cases(oracle):
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 1000.0, -1000.0, -1e9, 0.25], dtype=np.float32)
    # scale 1, zero point 0: ties to even, clamp at the int8 bounds (-1e9 saturates)
    assert oracle.quantize(x, oracle.F32, [1.0], [0], None, oracle.I8).tolist() == [0, 2, 2, 0, -2, 127, -128, -128, 0]
    # zero point added after rounding: rint(0.5) + 3 = 3 (not rint(3.5) = 4)
    assert oracle.quantize(x, oracle.F32, [1.0], [3], None, oracle.I8).tolist()[:3] == [3, 5, 5]
    # uint8 clamps at 0 and 255; scale 0.25 -> 1/scale = 4 exactly
    assert oracle.quantize(x, oracle.F32, [0.25], [128], None, 6).tolist() == [130, 134, 138, 126, 122, 255, 0, 0, 129]
    # qint32: the zero point is added in float32 (torch's quantize_val), 2e9 - 7 rounds back to 2e9
    assert oracle.quantize(np.array([1e9], np.float32), oracle.F32, [0.5], [-7], None, oracle.I32).tolist() \
        == [2000000000]
    assert oracle.quantize(np.array([3e9, -3e9], np.float32), oracle.F32, [1.0], [0], None, oracle.I32).tolist() \
        == [2147483647, -2147483648]


@pytest.mark.parametrize("code,npdt", [(4, np.int8), (6, np.uint8), (5, np.int32)])
def test_dequantize_is_float_cast(oracle, code, npdt):
    """The reference's dequantize is self.to(float) (op_plugin/ops/v1r11/opapi/DequantizeKernelNpuOpApi.cpp:22-24)."""
    g = np.random.default_rng(4)
    info = np.iinfo(npdt)
    q = g.integers(info.min, info.max, size=3000, dtype=np.int64, endpoint=True).astype(npdt)
    q[:4] = [info.min, info.max, 0, 1 if info.min == 0 else -1]
    assert np.array_equal(oracle.dequantize(q, code), torch.from_numpy(q).float().numpy())
