"""Shared helpers for the GPU parity tests: seeded synthetic tensors (the
same bytes go to the oracle and to the device), device transfers through
torch, and the reference-style tolerance check."""
import numpy as np

from oracle.oracle_py import Q8_DTYPE

QK = 32


def torch_cuda():
    import torch
    assert torch.cuda.is_available(), "GPU test without a GPU"
    return torch


# Device tensors made by dev() stay referenced until the test ends: a
# temporary freed right after its address is taken would let torch's caching
# allocator hand the same block to the next tensor before the kernel runs.
KEEP = []


def dev(a):
    torch = torch_cuda()
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    KEEP.append(t)
    return t


def empty(shape, dtype):
    torch = torch_cuda()
    t = torch.empty(shape, dtype=dtype, device="cuda")
    KEEP.append(t)
    return t


def zeros(shape, dtype):
    torch = torch_cuda()
    t = torch.zeros(shape, dtype=dtype, device="cuda")
    KEEP.append(t)
    return t


def dequant_q4(w_rowmajor, n, k):
    """float64 [n][k] values of row-major Q4_0 bytes."""
    b = np.asarray(w_rowmajor, np.uint8).reshape(n, k // 32, 18)
    d = b[:, :, :2].copy().view(np.uint16)[..., 0].view(np.float16).astype(np.float64)
    nib = np.concatenate([b[:, :, 2:] & 15, b[:, :, 2:] >> 4], axis=2).astype(np.float64) - 8
    return (nib * d[:, :, None]).reshape(n, k)


def dequant_q8(blocks, rows, k):
    """float64 [rows][k] values of block_q8_0 records."""
    q = blocks["qs"].astype(np.float64).reshape(rows, k // 32, 32)
    d = blocks["d"].view(np.float16).astype(np.float64).reshape(rows, k // 32, 1)
    return (q * d).reshape(rows, k)


class _DeviceArray:
    """__cuda_array_interface__ wrapper so torch can alias a raw device pointer."""

    def __init__(self, addr, count, typestr):
        self.__cuda_array_interface__ = {"shape": (count,), "typestr": typestr,
                                         "data": (int(addr), False), "version": 2}


def device_view(addr, count, dtype):
    """torch tensor aliasing count elements at a raw device address."""
    torch = torch_cuda()
    typestr = {torch.float32: "<f4", torch.int8: "|i1", torch.int16: "<i2",
               torch.int32: "<i4", torch.uint8: "|u1"}[dtype]
    return torch.as_tensor(_DeviceArray(addr, count, typestr), device="cuda")


def host(t):
    torch = torch_cuda()
    torch.cuda.synchronize()
    return t.cpu().numpy()


def close(got, want, rtol, what=""):
    """|a-b| <= atol + rtol*max(|a|,|b|) with atol = rtol*rms(want)
    (verify_fused_projections.c:39 form; rms-tied atol makes the relative
    test well posed near zero)."""
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape, (got.shape, want.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    rms = np.sqrt(np.mean(want ** 2)) if want.size else 0.0
    tol = rtol * rms + rtol * np.maximum(np.abs(got), np.abs(want))
    bad = np.abs(got - want) > tol
    if bad.any():
        i = int(np.argmax(np.abs(got - want) - tol))
        raise AssertionError(f"{what}: {bad.sum()}/{got.size} outside rtol {rtol} "
                             f"(worst i={i} got={got[i]:.7g} want={want[i]:.7g} rms={rms:.4g})")
    assert np.count_nonzero(want) > 0, f"{what}: reference all zero"


def planar_to_aos(qs, d):
    """planar Q8 (int8 [n*32], uint16 [n]) -> block_q8_0 records."""
    qs = np.asarray(qs, np.int8).reshape(-1, QK)
    out = np.zeros(qs.shape[0], Q8_DTYPE)
    out["qs"] = qs
    out["d"] = np.asarray(d, np.uint16).reshape(-1)
    return out


def aos_to_planar(blocks):
    return blocks["qs"].reshape(-1).copy(), blocks["d"].copy(), \
        blocks["qs"].astype(np.int32).sum(1).astype(np.int16)


def q8_tiled(qs, d, m, k):
    """Planar Q8 (int8 [m*k], uint16 [m*k/32]) -> operand-tiled (int8 and
    uint16 flat arrays): rows in ceil(m/32) panels of 32 (padding rows zero);
    block b of panel p is [half g][row j][16 bytes], half g of row j holding
    the block's bytes 8g..8g+7 then 16+8g..16+8g+7; scales [p][b][j]."""
    nb, P = k // QK, (m + 31) // 32
    a = np.zeros((P * 32, nb, QK), np.int8)
    a[:m] = np.asarray(qs, np.int8).reshape(m, nb, QK)
    sc = np.zeros((P * 32, nb), np.uint16)
    sc[:m] = np.asarray(d, np.uint16).reshape(m, nb)
    a = a.reshape(P, 32, nb, QK).transpose(0, 2, 1, 3)  # [p][b][j][32 bytes]
    halves = np.stack([np.concatenate([a[..., 0:8], a[..., 16:24]], -1),
                       np.concatenate([a[..., 8:16], a[..., 24:32]], -1)], 2)  # [p][b][g][j][16]
    td = sc.reshape(P, 32, nb).transpose(0, 2, 1)  # [p][b][j]
    return np.ascontiguousarray(halves).reshape(-1), np.ascontiguousarray(td).reshape(-1)


def q4(oracle, rng, n, k, sigma=0.02):
    return oracle.quantize_q4_0(rng.normal(0, sigma, (n, k)).astype(np.float32))


def make_layer(oracle, shape, seed, ffn=True, norm=True, bias=True):
    """Weights N(0,0.02) -> Q4_0, biases N(0,0.02), gains N(1,0.1)."""
    rng = np.random.default_rng(seed)
    H, QD, KVD, F = shape.hidden, shape.qheads * shape.hdim, shape.kvheads * shape.hdim, shape.ffn
    t = dict(wq=q4(oracle, rng, QD, H), wk=q4(oracle, rng, KVD, H), wv=q4(oracle, rng, KVD, H),
             wo=q4(oracle, rng, H, QD),
             norm=rng.normal(1, 0.1, H).astype(np.float32) if norm else None,
             bq=rng.normal(0, 0.02, QD).astype(np.float32) if bias else None,
             bk=rng.normal(0, 0.02, KVD).astype(np.float32) if bias else None,
             bv=rng.normal(0, 0.02, KVD).astype(np.float32) if bias else None)
    if ffn:
        t.update(post_norm=rng.normal(1, 0.1, H).astype(np.float32) if norm else None,
                 wgate=q4(oracle, rng, F, H), wup=q4(oracle, rng, F, H),
                 wdown=q4(oracle, rng, H, F))
    return t


def kv_history(oracle, rng, rows, kvd, scale=1.0):
    """N(0,1)*scale fp16 cache rows (RNE), as bits."""
    return oracle.f32_to_f16((rng.standard_normal(rows * kvd) * scale).astype(np.float32))
