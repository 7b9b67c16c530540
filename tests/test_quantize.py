"""Per-token 1x128 e4m3 quantization of the hidden states (the step before the operator).

Bar: codes and scales bit-exact with the oracle's arithmetic (scale = fp32(amax / 448),
1 for an all-zero block; codes = e4m3fn(fp32(x / scale)) rounded to nearest even).  The
oracle itself is pinned here against a brute-force encoder over the 256-code table.
"""
import numpy as np
import pytest
import torch

import moe_oracle as O


def sample(T, H, seed, dtype=torch.float32):
    """Rows of N(0,1) with per-row amplitudes from 1e-4 to 1e4, one all-zero 128-block, a
    negative zero, and values on e4m3 rounding midpoints after scaling."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g)
    amp = torch.logspace(-4, 4, T)
    x = x * amp[torch.randperm(T, generator=g)].unsqueeze(1)
    if T > 1 and H >= 256:
        x[1, 128:256] = 0.0
        x[1, 130] = -0.0
    if T > 2:
        # block max 448 -> scale 1 exactly, then midpoints between neighbouring e4m3 values
        x[2, :128] = 0.0
        x[2, 0] = 448.0
        x[2, 1:9] = torch.tensor([1.0625, 1.1875, -1.0625, 3 * 2.0**-10, -(2.0**-10), 0.9375 * 2.0**-6, 2.25, 464.0 - 16])
    return x.to(dtype)


def hard_scales(T, H, seed, dtype=torch.float32):
    """Blocks whose scales stress the division: block maxima with all-ones mantissas, exact
    powers of two, values just above/below them, tiny (near the fp32 normal minimum) and
    huge magnitudes, each block filled with random multiples of the maximum."""
    g = torch.Generator().manual_seed(seed)
    nb = H // 128
    maxes = []
    for k in range(T * nb):
        kind = k % 6
        e = int(torch.randint(-60, 60, (1,), generator=g))
        if kind == 0:
            m = (2.0 - 2.0**-23) * 2.0**e            # all-ones mantissa
        elif kind == 1:
            m = 2.0**e
        elif kind == 2:
            m = 2.0**e * (1 + 2.0**-23)
        elif kind == 3:
            m = 2.0**e * (1 - 2.0**-24)
        elif kind == 4:
            m = 2.0**-120 * float(torch.rand(1, generator=g) + 1)   # scale below 2^-100 (slow path)
        else:
            m = float(torch.rand(1, generator=g) + 0.5) * 2.0**int(torch.randint(-30, 30, (1,), generator=g))
        maxes.append(m)
    mx = torch.tensor(maxes, dtype=torch.float64).view(T, nb, 1)
    frac = torch.rand(T, nb, 128, generator=g, dtype=torch.float64) * 2 - 1
    frac[:, :, 0] = 1.0
    return (frac * mx).view(T, H).to(torch.float32).to(dtype)


# ------------------------------------------------------------------------------------------ CPU: oracle


@pytest.mark.parametrize("T,H,seed", [(7, 384, 1), (3, 256, 2), (16, 128, 3)])
def test_oracle_matches_bruteforce_encoder(T, H, seed):
    x = sample(T, H, seed)
    codes, scale = O.quantize_hidden(x)
    xb = x.view(T, H // 128, 128)
    amax = xb.abs().amax(dim=2).numpy()
    want_scale = np.where(amax > 0, (amax / np.float32(448.0)).astype(np.float32), np.float32(1.0))
    assert np.array_equal(scale, want_scale.T)
    v = (xb / torch.from_numpy(scale.T.copy()).unsqueeze(-1)).reshape(-1).numpy()
    assert np.array_equal(codes.reshape(-1), O.encode_e4m3_bruteforce(v))


def test_oracle_block_max_lands_on_448_and_zero_blocks():
    x = sample(9, 512, 4)
    codes, scale = O.quantize_hidden(x)
    vals = O.decode_e4m3(codes).reshape(9, 4, 128)
    amax = x.view(9, 4, 128).abs().amax(dim=2).numpy()
    nz = amax > 0
    assert np.all(np.abs(vals).max(axis=2)[nz] == 448.0)
    assert np.all(scale.T[~nz] == 1.0) and np.all(np.abs(vals)[~nz] == 0.0)
    # relative error of a nonzero normal value is at most half an e4m3 ulp (2^-4)
    deq = vals * scale.T[:, :, None]
    xr = x.view(9, 4, 128).numpy()
    normal = np.abs(xr) >= scale.T[:, :, None] * 2.0**-6
    assert np.all(np.abs(deq - xr)[normal] <= np.abs(xr)[normal] * 2.0**-4 * (1 + 1e-6))


def test_oracle_round_trip_of_representable_values():
    # blocks whose values are exact e4m3 values times a power-of-two scale quantize back to
    # the same codes
    rng = np.random.default_rng(5)
    finite = np.array([c for c in range(256) if np.isfinite(O.E4M3_TABLE[c])], dtype=np.uint8)
    codes = rng.choice(finite, size=(4, 256))
    codes[:, 0] = 0x7E                                   # block max 448 -> scale = 2^k exactly
    codes[:, 128] = 0xFE
    x = O.decode_e4m3(codes).astype(np.float32) * np.float32(2.0**-3)
    got, scale = O.quantize_hidden(torch.from_numpy(x))
    assert np.all(scale == np.float32(2.0**-3))
    assert np.array_equal(got, codes)


# ------------------------------------------------------------------------------------------ GPU: HIP path

DEV = torch.device("cuda:0")


@pytest.mark.gpu
@pytest.mark.parametrize("T,H,dtype", [(1, 7168, torch.bfloat16), (16, 7168, torch.bfloat16),
                                       (37, 384, torch.bfloat16), (64, 256, torch.float32),
                                       (300, 7168, torch.float32), (17, 640, torch.bfloat16)])
def test_quantize_bitexact(T, H, dtype):
    import moe_fp8
    print(f"[quantize] T={T} H={H} {dtype}", flush=True)
    x = sample(T, H, 10 + T, dtype)
    q, scale = moe_fp8.quantize_hidden(x.to(DEV))
    torch.cuda.synchronize()
    want_codes, want_scale = O.quantize_hidden(x)
    assert q.dtype == torch.float8_e4m3fn and tuple(q.shape) == (T, H)
    assert tuple(scale.shape) == (H // 128, T)
    assert np.array_equal(scale.cpu().numpy(), want_scale)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), want_codes)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_hard_scales(dtype):
    import moe_fp8
    print(f"[quantize] hard scales {dtype}", flush=True)
    x = hard_scales(512, 1024, 21, dtype)
    q, scale = moe_fp8.quantize_hidden(x.to(DEV))
    torch.cuda.synchronize()
    want_codes, want_scale = O.quantize_hidden(x)
    assert np.array_equal(scale.cpu().numpy(), want_scale)
    got = q.view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, want_codes), f"{int((got != want_codes).sum())} codes differ"


@pytest.mark.gpu
def test_quantize_full_size_t8192():
    import moe_fp8
    print("[quantize] T=8192 H=7168 bf16", flush=True)
    x = sample(8192, 7168, 11, torch.bfloat16)
    q, scale = moe_fp8.quantize_hidden(x.to(DEV))
    torch.cuda.synchronize()
    want_codes, want_scale = O.quantize_hidden(x)
    assert np.array_equal(scale.cpu().numpy(), want_scale)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), want_codes)


@pytest.mark.gpu
@pytest.mark.parametrize("T,H", [(65535 * 8 + 37, 128), (65535 * 8 * 2 + 8, 384)])
def test_quantize_more_token_groups_than_grid_rows(T, H):
    """A launch holds at most 65535 groups of 8 tokens: later groups are reached by striding, the
    last one partial."""
    import moe_fp8
    print(f"[quantize] T={T} H={H} bf16 (strided token groups)", flush=True)
    x = sample(T, H, 13, torch.bfloat16)
    q, scale = moe_fp8.quantize_hidden(x.to(DEV))
    torch.cuda.synchronize()
    want_codes, want_scale = O.quantize_hidden(x)
    assert np.array_equal(scale.cpu().numpy(), want_scale)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), want_codes)


@pytest.mark.gpu
def test_quantize_feeds_run():
    """The quantizer's output is the operator's input: run() on it equals run() on the
    oracle's quantization of the same activations, bit for bit."""
    import moe_fp8
    from moe_fp8 import workloads as W
    print("[quantize] feeds run T=16", flush=True)
    g = torch.Generator().manual_seed(12)
    T, E, H, I = 16, 8, 512, 256
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, 256, generator=g)
    bias = (torch.randn(256, generator=g) * 0.1).to(torch.bfloat16)
    w13, s13, w2, s2 = W.make_weights(E_local=E, H=H, I=I, seed=7)
    q, scale = moe_fp8.quantize_hidden(x.to(DEV))
    codes, sc = O.quantize_hidden(x)
    args = [logits.to(DEV), bias.to(DEV), None, None, w13.to(DEV), s13.to(DEV), w2.to(DEV), s2.to(DEV), 0, 2.5]
    out_a = moe_fp8.run(*args[:2], q, scale, *args[4:])
    out_b = moe_fp8.run(*args[:2], torch.from_numpy(codes).view(torch.float8_e4m3fn).to(DEV),
                        torch.from_numpy(sc).to(DEV), *args[4:])
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))


@pytest.mark.gpu
def test_quantize_rejects_bad_inputs():
    import moe_fp8
    with pytest.raises(ValueError):
        moe_fp8.quantize_hidden(torch.zeros(4, 100, device=DEV, dtype=torch.bfloat16))
    with pytest.raises(TypeError):
        moe_fp8.quantize_hidden(torch.zeros(4, 128, device=DEV, dtype=torch.float16))
    q, s = moe_fp8.quantize_hidden(torch.zeros(0, 128, device=DEV, dtype=torch.bfloat16))
    assert q.shape == (0, 128) and s.shape == (1, 0)
