"""GPU: the timing entry points - per-pass event times of a fit loop, and the streaming-read probe."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_per_pass_times_cover_every_pass():
    """One time per pass, across the host's batch boundaries; none while timing is off; cleared by profile(True)."""
    from mlx_kmeans import _lib
    rng = np.random.default_rng(3)
    X = rng.standard_normal((200_000, 32)).astype(np.float32)
    ctx = _lib.Context()
    ctx.set_parts([X])
    C0 = X[:64].copy()
    ctx.fit(C0, 5, -1.0)
    assert len(ctx.profile_passes()) == 0
    ctx.profile(True)
    _, _, n_iter, _ = ctx.fit(C0, 21, -1.0)
    t = ctx.profile_passes()
    assert n_iter == 21 and len(t) == 21
    assert np.all(t > 0.0) and np.all(t < 1e3)
    prof = ctx.profile_read()
    kernel_ms = sum(v[0] for v in prof.values())
    assert kernel_ms <= t.sum() * 1.05      # the kernels run inside the passes
    ctx.profile(True)
    assert len(ctx.profile_passes()) == 0
    ctx.profile(False)
    ctx.close()


def test_stream_probe_reads_at_a_plausible_rate():
    """The probe's best grid reads 1 GiB at between 1 TB/s and the 8 TB/s published peak; bad sizes are refused."""
    from mlx_kmeans import _lib
    ctx = _lib.Context()
    g = ctx.stream_probe(1 << 30, 5)
    print(f"[gpu] streaming read {g:.1f} GB/s", flush=True)
    assert 1000.0 < g < 8000.0
    with pytest.raises(ValueError):
        ctx.stream_probe((1 << 30) + 4, 5)
    with pytest.raises(ValueError):
        ctx.stream_probe(1 << 20, 5)
    ctx.close()
