"""The allocation-free decode entry point, dsv41_sparse_mla_decode_noalloc, called through the C
ABI: on the same inputs it must give dsv41_sparse_mla_decode's output and ring write (given a
caller workspace) bit for bit -- the same kernels read the same partials, only their home
differs. Two calls in a row, the second with a smaller batch and a shorter list, so the second
reads the static scratch the first left behind; a shape whose split scratch exceeds the static
32 MiB is refused on the host before any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from common import SEED_BASE

pytestmark = pytest.mark.gpu

H, D, RD, W = 64, 512, 64, 128


def _inputs(gen, device, b, nb, k, start):
    """bf16 q / ring / chunk / compressed cache N(0,1)/sqrt(576), sinks N(0,1), and a top-k list
    of each row's random scores (ascending, offset by the window, a few masked)."""
    from dsv41 import _abi
    s = 576 ** -0.5
    rn = lambda *shape: torch.randn(*shape, generator=gen, device=device)   # noqa: E731
    t = dict(q=(rn(b, 1, H, D) * s).bfloat16(), win=(rn(b, W, D) * s).bfloat16(), chunk=(rn(b, 1, D) * s).bfloat16(),
             comp=(rn(b, nb, D) * s).bfloat16(), sink=rn(H))
    scores = rn(b, 1, nb)
    t["idx"] = _abi.topk_select(scores, k, start, 4, min(start, W) + 1)
    return t


def _decode(name, t, start, cos, sin, ring, out, workspace=None):
    from dsv41 import _abi
    lib = _abi.lib()
    b, nb, k = t["comp"].shape[0], t["comp"].shape[1], t["idx"].shape[-1]
    p = lambda x: ctypes.c_void_p(x.data_ptr())   # noqa: E731
    args = [p(t["q"]), p(ring), p(t["chunk"]), p(t["comp"]), nb * D, nb, p(t["sink"]), p(t["idx"]), k, p(out), b, H, D,
            W, start, ctypes.c_float(D ** -0.5), p(cos), p(sin), RD, 0, _abi.BF16]
    if workspace is not None:
        args += [p(workspace), workspace.numel()]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = getattr(lib, name)(*args, stream)
    assert rc == 0, (name, rc, lib.dsv41_last_error_string())


def test_noalloc_decode_equals_the_workspace_form(gpu):
    from dsv41 import _abi
    from dsv41.layers import precompute_freqs_cis
    gen = torch.Generator(device=gpu).manual_seed(SEED_BASE + 90)
    cases = [(32, 16384, 512, 65535), (4, 2048, 256, 8200)]     # the second: fewer rows, shorter lists
    for b, nb, k, start in cases:
        print(f"[noalloc] b={b} nb={nb} k={k} start={start}", flush=True)
        t = _inputs(gen, gpu, b, nb, k, start)
        need = _abi.mla_workspace_bytes(b, 1, H, D, W + k, torch.bfloat16)
        assert 0 < need <= 32 << 20                                # the split path, inside the static buffer
        cos, sin = precompute_freqs_cis(RD, start + 1, 65536, 160000.0, 16.0, 32, 1, device=gpu)
        ring_ws, ring_na = t["win"].clone(), t["win"].clone()
        out_ws = torch.full_like(t["q"], float("nan"))
        out_na = torch.full_like(t["q"], float("nan"))
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        _decode("dsv41_sparse_mla_decode", t, start, cos, sin, ring_ws, out_ws, ws)
        _decode("dsv41_sparse_mla_decode_noalloc", t, start, cos, sin, ring_na, out_na)
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), (b, nb, k)
        assert torch.equal(ring_na, ring_ws), (b, nb, k)
        assert torch.equal(ring_na[:, start % W], t["chunk"][:, 0])   # the token landed in its slot


def test_noalloc_refuses_shapes_beyond_the_static_buffer(gpu):
    from dsv41 import _abi
    lib = _abi.lib()
    b, k = 128, 8192                       # 128 rows x 4 splits x 64 heads of partials: 32.25 MiB
    assert _abi.mla_workspace_bytes(b, 1, H, D, W + k, torch.bfloat16) > 32 << 20
    fake = ctypes.c_void_p(256)            # never dereferenced: refused before any launch
    rc = lib.dsv41_sparse_mla_decode_noalloc(fake, fake, fake, fake, 16384 * D, 16384, fake, fake, k, fake, b, H, D,
                                             W, 65535, ctypes.c_float(D ** -0.5), fake, fake, RD, 0, _abi.BF16,
                                             None)
    assert rc == -4 and b"static" in lib.dsv41_last_error_string()
