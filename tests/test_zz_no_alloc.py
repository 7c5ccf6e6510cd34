"""tris_backbone_linear_noalloc (the backbone projection with its split-K partial sums in a static device
array, for callers that cannot allocate) against tris_backbone_linear with a workspace, through the C ABI:
bit-identical outputs on calls in a row (decode-shaped kernel, then the tiled GEMM of a 512-row batch, then a
smaller decode batch), and a prefill shape whose partial sums exceed the array is rejected."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def test_backbone_noalloc_matches_workspace_entry(tris, cuda):
    from tris_moe_amd import _lib

    lib = _lib.load()
    ext = tris["ext"]
    assert lib.tris_backbone_noalloc_scratch_bytes() == 4 << 20
    rng = np.random.default_rng(71)
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    # (tokens, in, rank, gathered rows, input scale): the second call is smaller than the first
    cases = [(32, 4096, 512, True, True), (512, 1024, 128, False, True), (3, 1024, 256, False, False)]
    for tokens, in_f, rank, gather, scaled in cases:
        print(f"[gpu-case] backbone noalloc tokens={tokens} in={in_f} rank={rank}", flush=True)
        x = torch.from_numpy(rng.standard_normal((tokens, in_f)).astype(np.float16)).to(cuda)
        sv = torch.from_numpy((rng.standard_normal((rank, in_f)) * 0.02).astype(np.float16)).to(cuda)
        sc = torch.from_numpy(rng.uniform(0.5, 1.5, in_f).astype(np.float16)).to(cuda) if scaled else None
        rows = torch.from_numpy(rng.integers(0, tokens, 2 * tokens)).to(cuda) if gather else None
        n = 2 * tokens if gather else tokens
        assert lib.tris_backbone_workspace_bytes(n, in_f, rank) > 0  # the split-K path, which uses the scratch
        want = ext.backbone_linear(x, sv, in_scale=sc, row_index=rows)
        got = torch.full((n, rank), float("nan"), dtype=torch.float16, device=cuda)
        # tokens: the rows projected (row_index entries when gathering), as tris_backbone_linear takes it
        rc = lib.tris_backbone_linear_noalloc(_ptr(x), n, in_f, _ptr(rows), _ptr(sv), rank, _ptr(sc),
                                              _ptr(got), stream)
        assert rc == 0, lib.tris_last_error()
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_backbone_noalloc_rejects_oversized_scratch(tris, cuda):
    """512 x 4096 -> 512 takes the tiled GEMM with 8 slices (8 MiB of partial sums): rejected with an error that
    names the workspace entry, and nothing is written."""
    from tris_moe_amd import _lib

    lib = _lib.load()
    tokens, in_f, rank = 512, 4096, 512
    assert lib.tris_backbone_workspace_bytes(tokens, in_f, rank) > lib.tris_backbone_noalloc_scratch_bytes()
    x = torch.zeros((tokens, in_f), dtype=torch.float16, device=cuda)
    sv = torch.zeros((rank, in_f), dtype=torch.float16, device=cuda)
    out = torch.full((tokens, rank), 7.0, dtype=torch.float16, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    rc = lib.tris_backbone_linear_noalloc(_ptr(x), tokens, in_f, None, _ptr(sv), rank, None, _ptr(out), stream)
    assert rc == -1
    assert b"tris_backbone_linear with a workspace" in lib.tris_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
