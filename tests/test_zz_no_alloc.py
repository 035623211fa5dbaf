"""mamba2_stack_step_noalloc (the allocation-free decode stack step, its
workspace a per-GPU file-scope device array) against mamba2_stack_step with a
caller workspace: two calls in a row through the C ABI, the second at a
smaller batch, each compared with the workspace entry point on identical
inputs and caches (same kernels, so identical results)."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _stack_args(stack, x, caches):
    import mamba_hip
    from mamba_hip import _lib
    del mamba_hip
    return (_lib.Mamba2LayerArgs * len(stack.layers))(
        *[stack._layer_args(i, x, caches[i]) for i in range(len(stack.layers))])


def _one(stack, b, seed):
    import torch
    import mamba_hip
    from mamba_hip import _lib
    from mamba_hip.ssd import _stream
    L = _lib.lib()
    c = stack.cfg
    gen = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn((b, c.d_model), generator=gen, device="cuda")
    caches = stack.new_caches(b)
    for cc in caches:
        cc.ssm_bhpr.normal_(0.0, 0.1, generator=gen)
        cc.conv_bvk.normal_(0.0, 1.0, generator=gen)
    x2 = x.clone()
    caches2 = [mamba_hip.Mamba2Cache(cc.conv_bvk.clone(), cc.ssm_bhpr.clone()) for cc in caches]
    stream = _stream(x.device)
    a1 = _stack_args(stack, x, caches)
    print(f"noalloc stack step: {len(stack.layers)} layers, batch {b}", flush=True)
    assert L.mamba2_stack_step_noalloc(a1, len(stack.layers), stream) == 0, L.mamba_last_error()
    need = L.mamba2_layer_workspace_size(ctypes.byref(a1[0]))
    assert 0 < need <= (48 << 20)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    a2 = _stack_args(stack, x2, caches2)
    assert L.mamba2_stack_step(a2, len(stack.layers), ctypes.c_void_p(ws.data_ptr()), need, stream) == 0
    torch.cuda.synchronize()
    assert torch.isfinite(x).all()
    np.testing.assert_array_equal(x.cpu().numpy(), x2.cpu().numpy())
    for p, q in zip(caches, caches2):
        np.testing.assert_array_equal(p.ssm_bhpr.cpu().numpy(), q.ssm_bhpr.cpu().numpy())
        np.testing.assert_array_equal(p.conv_bvk.cpu().numpy(), q.conv_bvk.cpu().numpy())


def test_stack_step_noalloc_matches_workspace_entry_point():
    import torch
    import mamba_hip
    cfg = mamba_hip.Mamba2Config(d_model=512)
    stack = mamba_hip.Mamba2Stack.init(cfg, 3, "cuda", torch.bfloat16, torch.Generator().manual_seed(8), fused=True)
    assert stack.fused
    _one(stack, 64, 1)   # first call: the scratch address is looked up
    _one(stack, 5, 2)    # second call, smaller batch: the array keeps the last call's contents


def test_stack_step_noalloc_rejects_oversize():
    """A stack needing more workspace than the 48 MiB scratch array (16 groups
    at d_model 4096, batch 256: 54 MiB) is refused with MAMBA_ERR_WORKSPACE
    before any launch; the pointers are never dereferenced, so placeholders
    stand in for them."""
    from mamba_hip import _lib
    L = _lib.lib()
    a = (_lib.Mamba2LayerArgs * 1)()
    a[0].batch, a[0].d_model, a[0].nheads, a[0].headdim = 256, 4096, 128, 64
    a[0].ngroups, a[0].dstate, a[0].conv_kernel = 16, 128, 4
    fake = 1 << 20
    a[0].x, a[0].x_sb, a[0].pre_norm_w, a[0].in_proj, a[0].out_proj = fake, 4096, fake, fake, fake
    a[0].ssm_state, a[0].conv_state, a[0].conv_w = fake, fake, fake
    assert L.mamba2_layer_workspace_size(ctypes.byref(a[0])) > (48 << 20)
    assert L.mamba2_stack_step_noalloc(a, 1, None) == 3  # MAMBA_ERR_WORKSPACE
    assert b"scratch" in L.mamba_last_error()
