"""Runtime behaviour at the C ABI: host -> device copies through the pinned staging ring keep
stream order and let the caller reuse its buffer at once, behind queued device work; queue marks
(anima_mark / anima_wait_mark) order correctly and reject tickets never issued; the device limits
(anima_device_limits) describe the MI355X."""

import ctypes

import numpy as np
import pytest

from helpers import amd

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def ctx():
    m = amd()
    c = m.Context(0)
    yield c
    c.close()


def queue_attention(ctx, m, reps):
    """Enqueue `reps` fused self-attention launches (B=2, 4096 tokens, 16 heads): ~0.3 ms each."""
    B, L, H, D = 2, 4096, 16, 128
    qkv = ctx.empty((B * L, 3 * H * D))
    ctx.fill_random(qkv, B * L * 3 * H * D, "f32", 7, -1.0, 1.0)
    o = ctx.empty((B * L, H * D))
    for _ in range(reps):
        ctx.attention(q=qkv, k=qkv, v=qkv, o=o, B=B, Lq=L, Lk=L, H=H, D=D, ldq=3 * H * D, ldk=3 * H * D,
                      ldv=3 * H * D, k_off=H * D, v_off=2 * H * D, q_bstride=L * 3 * H * D,
                      k_bstride=L * 3 * H * D, v_bstride=L * 3 * H * D, o_bstride=L * H * D)
    return qkv, o


def test_h2d_staging_order_and_source_reuse(ctx):
    """Twelve uploads (more than the ring's four slots, sizes up to the 4 MiB slot and one above it
    that takes the pageable path) from ONE host array rewritten after every call, behind ~6 ms of
    queued attention; a device copy enqueued before each upload must still see the old contents."""
    m = amd()
    lib = m.lib()
    sizes = [1, 3, 1000, 65536, 1 << 20, (1 << 20) + 1, 7, 250000, 1 << 20, 4096, 17, 123457]
    case(f"h2d staging: {len(sizes)} uploads of {sizes} floats behind 20 queued attention launches")
    bufs = [ctx.empty(n) for n in sizes]
    olds = [ctx.empty(n) for n in sizes]
    init = [np.full(n, -float(i + 1), np.float32) for i, n in enumerate(sizes)]
    for b, a in zip(bufs, init):
        b.write(a)
    ctx.sync()
    keep = queue_attention(ctx, m, 20)
    host = np.empty(max(sizes), np.float32)
    want = []
    for i, (b, old, n) in enumerate(zip(bufs, olds, sizes)):
        # the copy of the previous contents is enqueued first: it must read them, not the upload
        ctx._check(lib.anima_d2d(ctx.h, old.ptr, b.ptr, n * 4))
        host[:n] = np.arange(n, dtype=np.float32) * 0.5 + i
        want.append(host[:n].copy())
        ctx._check(lib.anima_h2d(ctx.h, b.ptr, host.ctypes.data, n * 4))
        host[:] = np.nan  # the caller may reuse its buffer as soon as the call returns
    for i, (b, old) in enumerate(zip(bufs, olds)):
        assert np.array_equal(b.numpy(), want[i]), f"upload {i} ({sizes[i]} floats)"
        assert np.array_equal(old.numpy(), init[i]), f"copy before upload {i}"
    for t in bufs + olds + list(keep):
        t.release()


def test_marks_order_and_errors(ctx):
    case("anima_mark / anima_wait_mark: tickets, waits behind queued work, old and unissued tickets")
    m = amd()
    t0 = ctx.mark()
    keep = queue_attention(ctx, m, 10)
    x = ctx.empty(1 << 16)
    ctx.fill_random(x, 1 << 16, "f32", 3, 0.0, 1.0)
    t1 = ctx.mark()
    assert t1 == t0 + 1
    ctx.wait_mark(t1)
    # the fill enqueued before t1 is in place
    host = np.empty(1 << 16, np.float32)
    ctx._check(m.lib().anima_d2h(ctx.h, host.ctypes.data, x.ptr, host.nbytes))
    assert np.all((host >= 0) & (host < 1))
    # more marks than the ring holds: an old ticket still waits (for a later point)
    ts = [ctx.mark() for _ in range(40)]
    ctx.wait_mark(ts[0])
    ctx.wait_mark(t0)
    with pytest.raises(m.AnimaError) as e:
        ctx.wait_mark(ts[-1] + 1)
    assert e.value.code == -1 and "not issued" in str(e.value)  # ANIMA_E_ARG
    # the context stays usable after the rejected call
    ctx.wait_mark(ts[-1])
    ctx.sync()
    for t in [x] + list(keep):
        t.release()


def test_device_limits(ctx):
    """anima_device_limits reports the device the context runs on: gfx950, 256 compute units,
    64-wide wavefronts, 288 GB of HBM as the buffer / binding bound, 160 KiB of LDS per workgroup
    at most, and a free-memory figure within the total."""
    case("device limits")
    L = ctx.limits()
    print(f"limits: {L}", flush=True)
    assert L["arch"].startswith("gfx950")
    assert L["compute_units"] == 256 and L["wavefront_size"] == 64
    assert L["max_buffer_size"] == L["max_binding_size"] >= 250 * 10**9
    assert 0 < L["free_memory"] <= L["total_memory"]
    assert 64 * 1024 <= L["workgroup_storage_size"] <= 160 * 1024
    assert L["max_workgroup_size"] >= 1024 and L["max_workgroups_per_dimension"] >= 65535
