"""anima_attention_noalloc (the allocation-free variant of anima_attention) through the C ABI:
bit-identical to anima_attention on two calls in a row (the second smaller, so the shared scratch
holds the first call's bytes when the second runs), no pool or workspace growth across its calls,
and a clear rejection of a K/V conversion larger than the scratch."""

import numpy as np
import pytest

import oracle as orc
from helpers import amd

pytestmark = pytest.mark.gpu

HD = 128


def qkv_case(seed, B, L, H):
    qkv = orc.randn(seed, B * L * 3 * H * HD).reshape(B, L, 3 * H * HD)
    qn = (1 + 0.02 * orc.randn(seed + 1, HD)).astype(np.float32)
    kn = (1 + 0.02 * orc.randn(seed + 2, HD)).astype(np.float32)
    Hp = int(np.sqrt(L))
    cs = orc.dit_rope_table(Hp, L // Hp)
    return qkv, qn, kn, cs


def test_noalloc_attention_matches_attention_twice():
    m = amd()
    assert m.Context.attention_noalloc_scratch_bytes() == 64 << 20
    with m.Context() as ctx:
        for precision in (m.PREC_BF16, m.PREC_FP32):
            cases = []
            # a large call (the 8-wave bf16 kernel) and then a smaller one (the 4-wave kernel)
            for seed, B, L, H in ((31, 2, 1024, 16), (41, 1, 256, 4)):
                qkv, qn, kn, cs = qkv_case(seed, B, L, H)
                d = [ctx.upload(a) for a in (qkv, qn, kn, cs)]
                ld = 3 * H * HD
                args = dict(q=d[0], k=d[0], v=d[0], B=B, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld, k_off=H * HD,
                            v_off=2 * H * HD, precision=precision, q_norm=d[1], k_norm=d[2], rope_cs=d[3],
                            rope_sin_off=L * (HD // 2))
                o1 = ctx.empty((B, L, H * HD))
                ctx.attention(o=o1, **args)
                cases.append((d, args, o1, (B, L, H)))
            outs = [ctx.empty(o1.shape) for _, _, o1, _ in cases]
            ctx.sync()
            before = ctx.mem_stats()
            for (d, args, o1, shape), o2 in zip(cases, outs):  # the two allocation-free calls in a row
                print(f"[case] noalloc B,L,H={shape} precision={precision}", flush=True)
                ctx.attention(o=o2, noalloc=True, **args)
            ctx.sync()
            after = ctx.mem_stats()
            assert after == before  # no pool or workspace growth
            for (d, args, o1, shape), o2 in zip(cases, outs):
                r1, r2 = o1.numpy(), o2.numpy()
                assert np.all(np.isfinite(r2))
                assert np.array_equal(r1, r2), (shape, precision)
                for x in d + [o1, o2]:
                    x.release()


def test_noalloc_attention_rejects_scratch_overflow():
    m = amd()
    with m.Context() as ctx:
        # B=2, 16 heads, N=4096 in fp32 needs 128 MiB of K/V scratch (the inputs are real buffers of
        # that shape; the call is refused before any launch)
        B, L, H = 2, 4096, 16
        need = m.Context.attention_kv_bytes(B, H, L, m.PREC_FP32)
        assert need == 128 << 20
        qkv = ctx.empty((B, L, 3 * H * HD))
        ctx.fill_random(qkv, B * L * 3 * H * HD, "f32", 77, -1.0, 1.0)
        o = ctx.empty((B, L, H * HD))
        ld = 3 * H * HD
        with pytest.raises(m.AnimaError) as e:
            ctx.attention(q=qkv, k=qkv, v=qkv, o=o, B=B, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld, k_off=H * HD,
                          v_off=2 * H * HD, precision=m.PREC_FP32, noalloc=True)
        assert e.value.code == -1 and "maximum" in str(e.value)
        # the same shape in bf16 is exactly the maximum and runs
        assert m.Context.attention_kv_bytes(B, H, L, m.PREC_BF16) == 64 << 20
        ctx.attention(q=qkv, k=qkv, v=qkv, o=o, B=B, Lq=L, Lk=L, H=H, D=HD, ldq=ld, ldk=ld, ldv=ld, k_off=H * HD,
                      v_off=2 * H * HD, precision=m.PREC_BF16, noalloc=True)
        ctx.sync()
        qkv.release()
        o.release()
