"""lq_resident_attention_noalloc: decode attention whose counters and split
records live in the library's static device array instead of a caller
workspace (for callers that cannot allocate device memory).

* GPU: on calls in a row -- an 8-kv-head, group-4 step with an fp16 tail,
  then a smaller one, then the first geometry again (the array keeps the
  previous call's contents, so this also checks that every call leaves its
  completion counters at zero) -- its output and lq_resident_attention's
  (caller workspace) are both within the attention bar of the oracle's
  float64 attention (1e-3 of the head's largest output), and within 2 fp16
  ulps of each other elementwise: the kernel deals prefix tiles to waves
  dynamically, so two calls may sum in different orders.
* CPU: a step whose workspace exceeds LQ_RES_ATTN_SCRATCH_BYTES is refused
  with LQ_ERR_SCRATCH from the host-side geometry alone, before any HIP call
  (the struct's device pointers are never dereferenced).
"""
import ctypes

import numpy as np
import pytest
import torch

LQ_ERR_SCRATCH = -5
LQ_RES_ATTN_SCRATCH_BYTES = 4 << 20


def _resident(H, T, seed):
    from latticequant_amd.llm.resident import ResidentKV
    from oracle import oracle as O
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, H, T, 128, generator=g).half()
    ch = O.compress_chunk(x[0].numpy()[None], 4)
    r = ResidentKV(H, T, device="cuda")
    r.append(x.cuda(), torch.from_numpy(ch.scales_f32), torch.from_numpy(ch.scales.astype(np.float16)))
    return r


def _resident_ref(H, T, seed):
    """Resident prefix and the oracle's dequantised values (1, H, T, 128)."""
    from latticequant_amd.llm.resident import ResidentKV
    from oracle import oracle as O
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, H, T, 128, generator=g).half()
    ch = O.compress_chunk(x[0].numpy()[None], 4)
    r = ResidentKV(H, T, device="cuda")
    r.append(x.cuda(), torch.from_numpy(ch.scales_f32), torch.from_numpy(ch.scales.astype(np.float16)))
    return r, O.decompress_chunk(ch).reshape(1, H, T, 128)


def _both(H, T, group, Tt, seed):
    """(workspace output, no-alloc output, float64 oracle) of one step on fresh inputs."""
    from oracle import oracle as O
    from latticequant_amd import _lib as L
    from latticequant_amd.llm.resident import attn_workspace
    lib = L.lib()
    (k, kref), (v, vref) = _resident_ref(H, T, seed), _resident_ref(H, T, seed + 1)
    g = torch.Generator().manual_seed(seed + 2)
    q = torch.randn(H * group, 128, generator=g).half().cuda()
    tk = torch.randn(H, max(Tt, 1), 128, generator=g).half().cuda()
    tv = torch.randn(H, max(Tt, 1), 128, generator=g).half().cuda()
    ks, vs = k.struct(), v.struct()
    assert lib.lq_resident_attn_workspace(H, group, T, Tt) <= LQ_RES_ATTN_SCRATCH_BYTES
    work = attn_workspace(H, group, T, Tt, "cuda")
    ref = torch.empty(H * group, 128, dtype=torch.float16, device="cuda")
    out = torch.full_like(ref, float("nan"))
    s = L.stream_ptr()
    tkp, tvp = (tk.data_ptr(), tv.data_ptr()) if Tt > 0 else (None, None)
    rc = lib.lq_resident_attention(ctypes.addressof(ks), ctypes.addressof(vs), T, q.data_ptr(), group, tkp, tvp, Tt,
                                   work.data_ptr(), ref.data_ptr(), s)
    assert rc == 0, lib.lq_status_string(rc)
    rc = lib.lq_resident_attention_noalloc(ctypes.addressof(ks), ctypes.addressof(vs), T, q.data_ptr(), group, tkp,
                                           tvp, Tt, out.data_ptr(), s)
    assert rc == 0, lib.lq_status_string(rc)
    torch.cuda.synchronize()
    K = np.concatenate([kref, tk[:, :Tt].cpu().numpy()[None]], 2)
    V = np.concatenate([vref, tv[:, :Tt].cpu().numpy()[None]], 2)
    orc = O.decode_attention(q.cpu().numpy().reshape(1, H * group, 1, 128), K, V).reshape(H * group, 128)
    return ref.cpu().numpy(), out.cpu().numpy(), orc


def _head_err(o, r):
    return (np.abs(o.astype(np.float64) - r).max(1) / (np.abs(r).max(1) + 1e-30)).max()


@pytest.mark.gpu
def test_noalloc_attention_equals_workspace_entry_point_gpu():
    for (H, T, group, Tt, seed) in [(8, 8192, 4, 128, 0),     # C3's heads and group, 8192-token prefix
                                    (4, 1024, 8, 32, 10),     # smaller: fewer heads, splits, records
                                    (8, 8192, 4, 128, 20)]:   # the first geometry again, new inputs
        print(f"noalloc step H={H} T={T} group={group} tail={Tt} seed={seed}", flush=True)
        ref, out, orc = _both(H, T, group, Tt, seed)
        assert np.isfinite(ref).all() and np.isfinite(out).all()
        e_ws, e_na = _head_err(ref, orc), _head_err(out, orc)
        d = np.abs(out.astype(np.float32) - ref.astype(np.float32))
        ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32)
        print(f"  err vs oracle: workspace {e_ws:.2e} noalloc {e_na:.2e}; differing {int((d > 0).sum())} of {d.size}, "
              f"max diff {d.max():.3e} = {float((d / ulp).max()):.1f} ulp", flush=True)
        assert e_ws <= 1e-3 and e_na <= 1e-3
        assert (d <= 2 * ulp).all()


def test_noalloc_attention_refuses_oversize_step():
    """Refused from the geometry before any HIP call: the pointers are stand-ins."""
    from latticequant_amd import _lib as L
    lib = L.load()
    fake = ctypes.c_void_p(0x1000)
    H, group, T = 128, 16, 4096
    assert lib.lq_resident_attn_workspace(H, group, T, 0) > LQ_RES_ATTN_SCRATCH_BYTES
    r = L.Resident(a=fake, b=fake, mask=fake, meta=fake, exc=fake, scale=fake, n_exc=fake, status=fake,
                   n_heads=H, cap_blocks=T // 16, exc_cap=1)
    rc = lib.lq_resident_attention_noalloc(ctypes.addressof(r), ctypes.addressof(r), T, fake, group, None, None, 0,
                                           fake, None)
    assert rc == LQ_ERR_SCRATCH
    assert "scratch" in lib.lq_status_string(rc).decode()
