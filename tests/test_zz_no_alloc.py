"""difflet_rocm_attention_noalloc (the attention entry point that allocates nothing, its split
schedule's workspace a static device array of the library) against difflet_rocm_attention with
a caller workspace, both through the C ABI: equal outputs bit for bit (the same kernels and
schedule), on calls in a row whose second input is smaller, so the second call runs on what the
first left in the shared array."""

import ctypes
import math

import pytest
import torch

from difflet_amd import _lib

pytestmark = pytest.mark.gpu


def _arr(vals):
    return (ctypes.c_int64 * len(vals))(*vals)


def _call(fn, q, k, v, o, scale, ws=None, bounds=None, causal=False):
    b, h, sq, d = q.shape
    sk = k.shape[2]
    bmin = bmax = bstr = None
    if bounds is not None:
        bmin, bmax = (ctypes.c_void_p(t.data_ptr()) for t in bounds)
        bstr = _arr(bounds[0].stride())
    args = [ctypes.c_void_p(t.data_ptr()) for t in (q, k, v, o)]
    args += [_lib.BF16, b, h, sq, sk, d, _arr(q.stride()[:3]), _arr(k.stride()[:3]),
             _arr(v.stride()[:3]), _arr(o.stride()[:3]), float(scale), int(causal), None, 0,
             None, bmin, bmax, bstr]
    if ws is not None:
        args += [ctypes.c_void_p(ws.data_ptr()), ws.numel()]
    stream = ctypes.c_void_p(torch.cuda.current_stream(q.device).cuda_stream)
    st = fn(*args, stream)
    _lib.check(st, fn.__name__)


def _case(gpu, h, sq, sk, seed):
    g = torch.Generator(device=gpu).manual_seed(seed)
    mk = lambda s: torch.randn(1, h, s, 128, generator=g, device=gpu).to(torch.bfloat16)  # noqa: E731
    return mk(sq), mk(sk), mk(sk)


# FLUX's 24 x 4608 (split schedule), then a smaller split launch (20 x 2048), then a short
# unsplit one (whole tiles) and a key-bounded one (the masked kernel): the shared array keeps
# each call's contents for the next
CASES = [(24, 4608, 4608, None), (20, 2048, 2048, None), (2, 300, 700, None),
         (3, 513, 1088, "bounds")]


def test_noalloc_attention_equals_the_workspace_entry_point(gpu):
    lib = _lib.load()
    nbytes = int(lib.difflet_rocm_attention_workspace_bytes())
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    for i, (h, sq, sk, extra) in enumerate(CASES):
        print(f"noalloc attention call {i}: h={h} sq={sq} sk={sk} {extra or ''}", flush=True)
        q, k, v = _case(gpu, h, sq, sk, 100 + i)
        bounds = None
        if extra == "bounds":
            lo = torch.randint(0, sk // 2, (1, h, sq), device=gpu, dtype=torch.int32)
            hi = lo + torch.randint(1, sk // 2, (1, h, sq), device=gpu, dtype=torch.int32)
            bounds = (lo, hi)
        scale = 1 / math.sqrt(128)
        want = torch.empty_like(q)
        got = torch.full_like(q, float("nan"))
        _call(lib.difflet_rocm_attention, q, k, v, want, scale, ws=ws, bounds=bounds)
        _call(lib.difflet_rocm_attention_noalloc, q, k, v, got, scale, bounds=bounds)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}"
        # the caller's workspace counters are back at zero, as the contract says
        assert int(torch.count_nonzero(ws[:16384])) == 0
