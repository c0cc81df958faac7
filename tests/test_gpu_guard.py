"""Guard bands around every attention output. Each output (o, L, dq, dk, dv,
and the decode output and L) is a view into a larger buffer filled with a
sentinel: padded rows before and after the sequence, a padded row stride (so
each row is followed by unused elements), and padding around the (b, h)
slices. After the call every element outside the views must still hold the
sentinel, for the MFMA and the tiled kernels, forward and backward (plain,
masked, non-causal) and decode, at ragged lengths T in {1, 33, 333, 4097}.
The MFMA kernels stage through raw buffer loads and guard their stores per
row; these tests check that no store lands outside its row or sequence."""

import math

import pytest
import torch

import fastalgebraictransformer_amd as F
from fastalgebraictransformer_amd.backward import _attn_bwd_into
from fastalgebraictransformer_amd.forward import _attn_fwd_into, _key_mask_arg

pytestmark = pytest.mark.gpu
dev = "cuda"
PAD_T = 5      # sentinel rows before and after each (b, h) sequence
SENTINEL = -1234.5  # exact in bf16, fp16 and fp32


def _guarded(B, H, T, D, dtype, pad_d):
    """A [B, H, T, D] view (row stride D + pad_d) inside a sentinel buffer, and
    the buffer with a boolean map of the view's elements."""
    buf = torch.full((B, H + 1, T + 2 * PAD_T, D + pad_d), SENTINEL, dtype=dtype, device=dev)
    view = buf[:, :H, PAD_T:PAD_T + T, :D]
    inside = torch.zeros(buf.shape, dtype=torch.bool, device=dev)
    inside[:, :H, PAD_T:PAD_T + T, :D] = True
    return view, buf, inside


def _guarded_L(B, H, T):
    buf = torch.full((B, H + 1, T + 2 * PAD_T), SENTINEL, dtype=torch.float32, device=dev)
    inside = torch.zeros(buf.shape, dtype=torch.bool, device=dev)
    inside[:, :H, PAD_T:PAD_T + T] = True
    return buf[:, :H, PAD_T:PAD_T + T], buf, inside


def _untouched(buf, inside, name):
    torch.cuda.synchronize()
    outside = buf[~inside]
    bad = int((outside != SENTINEL).sum())
    assert bad == 0, f"{name}: {bad} elements written outside the view"


CASES = [(dt, impl) for dt in (torch.bfloat16, torch.float16) for impl in ("mfma", "tiled")] + \
        [(torch.float32, "tiled")]


@pytest.mark.parametrize("dtype,impl", CASES)
@pytest.mark.parametrize("T", [1, 33, 333, 4097])
@pytest.mark.parametrize("mode", ["plain", "masked", "noncausal"])
def test_attention_writes_stay_in_their_views(gpu, dtype, impl, T, mode, monkeypatch):
    if T == 4097 and impl == "tiled" and mode != "plain":
        pytest.skip("the long tiled case runs once (plain); masking does not change its stores")
    monkeypatch.setenv("KAT_ATTN_IMPL", impl)
    B, H, D = 2, 2, 64 if T == 4097 else 128
    pad_d = 8  # keeps 16-byte row alignment (MFMA path) while leaving a gap after every row
    g = torch.Generator().manual_seed(T + D)
    q, k, v, do = (torch.randn(B, H, T, D, generator=g).to(dtype).to(dev) for _ in range(4))
    slopes = F.compute_alibi_slopes(H).to(dev)
    scale = 1.0 / math.sqrt(D)
    km, causal, ext = None, True, False
    if mode != "plain":
        ext, causal = True, mode == "masked"
        m = torch.ones(B, T, dtype=torch.int32)
        m[0, : max(1, T // 3)] = 0
        m[1, 3::5] = 0
        km = _key_mask_arg(m, B, T, dev)
    o, obuf, oin = _guarded(B, H, T, D, dtype, pad_d)
    L, lbuf, lin = _guarded_L(B, H, T)
    _attn_fwd_into(q, k, v, o, L, slopes, scale, causal, 1e-6, km, extended=ext)
    _untouched(obuf, oin, "o")
    _untouched(lbuf, lin, "L")
    grads = [_guarded(B, H, T, D, dtype, pad_d) for _ in range(3)]
    dq, dk, dv = (gr[0] for gr in grads)
    _attn_bwd_into(q, k, v, o, L, do, dq, dk, dv, slopes, scale, causal, 1e-6, km, extended=ext)
    for name, (_, buf, inside) in zip(("dq", "dk", "dv"), grads):
        _untouched(buf, inside, name)
    for t in (o, L, dq, dk, dv):
        assert bool(torch.isfinite(t).all())


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.float16, 256), (torch.float32, 64)])
@pytest.mark.parametrize("T", [1, 33, 4097])
def test_decode_writes_stay_in_their_views(gpu, dtype, D, T):
    from fastalgebraictransformer_amd import _lib
    B, H = 3, 4
    g = torch.Generator().manual_seed(T + D + 1)
    q = torch.randn(B, H, D, generator=g).to(dtype).to(dev)
    kc = torch.randn(B, T, H, D, generator=g).to(dtype).to(dev).permute(0, 2, 1, 3)
    vc = torch.randn(B, T, H, D, generator=g).to(dtype).to(dev).permute(0, 2, 1, 3)
    slopes = F.compute_alibi_slopes(H).to(dev)
    obuf = torch.full((B, H + 1, D + 8), SENTINEL, dtype=dtype, device=dev)
    oin = torch.zeros(obuf.shape, dtype=torch.bool, device=dev)
    oin[:, :H, :D] = True
    out = obuf[:, :H, :D]
    lbuf = torch.full((B * H + 2 * PAD_T,), SENTINEL, dtype=torch.float32, device=dev)
    lin = torch.zeros(lbuf.shape, dtype=torch.bool, device=dev)
    lin[PAD_T:PAD_T + B * H] = True
    L = lbuf[PAD_T:PAD_T + B * H]
    lengths = torch.tensor([T, max(0, T - 7), T // 2], dtype=torch.int32, device=dev)
    lib = _lib.load()
    code = _lib.dtype_code(q)
    ws_bytes = lib.kat_attn_decode_workspace_size(B, H, T, D, code)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    strides = _lib.i64_array((q.stride(0), q.stride(1), kc.stride(0), kc.stride(1), kc.stride(2),
                              vc.stride(0), vc.stride(1), vc.stride(2), out.stride(0), out.stride(1)))
    _lib.check(lib.kat_attn_decode(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                                   L.data_ptr(), slopes.data_ptr(), lengths.data_ptr(), ws.data_ptr(),
                                   ws_bytes, B, H, T, D, strides, 0.1, 1e-6, code, _lib.stream(q)),
               "kat_attn_decode")
    _untouched(obuf, oin, "decode out")
    _untouched(lbuf, lin, "decode L")
    assert bool(torch.isfinite(out).all())
