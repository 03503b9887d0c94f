"""allie_extend_noalloc against allie_extend, through the C ABI.

The allocation-free entry point runs the same kernels over the library's
per-device scratch instead of a caller workspace, so its outputs must equal
allie_extend's bit for bit.  Two calls in a row, the second smaller (the
scratch keeps the first call's contents), on the tiny model in each mode
(bf16: fan-kernel groups, then one-token decode groups; fp8 weights, whose
GEMMs widen the e4m3 bytes in registers here instead of in the workspace;
the fp32 check mode), on the medium model at the 256-token maximum (one
token more is rejected before any launch), and on the 2x fp8 shape at the
maximum, which must fit the scratch.
"""
import numpy as np
import pytest
import torch

from allie_amd import capi, config, weights
from allie_amd.engine import Engine

pytestmark = pytest.mark.gpu

FIELDS = ("logits", "value", "time", "top1", "max_logit", "lse")


def roots(eng, n_roots, prefix_len, seed):
    """Prefill n_roots games of prefix_len ids into a fresh pool; returns
    (pool, root block table [R, nb], first free block)."""
    rng = np.random.default_rng(seed)
    nb = -(-prefix_len // 16)
    ids = rng.integers(0, 1968, (n_roots, prefix_len)).astype(np.uint32)
    table = torch.arange(n_roots * nb, dtype=torch.int32, device=eng.device).reshape(n_roots, nb)
    pool = eng.new_kv_pool(n_roots * nb + 64).zero_()  # ancestors' slots below are read, never written
    wd = torch.from_numpy(ids.reshape(-1).view(np.int32)).to(eng.device)
    eng.prefill(wd, np.full(n_roots, prefix_len, np.int32), kv_pool=pool, kv_block_table=table, want_logits=False)
    return pool, table, n_roots * nb


def batch(rng, table, prefix_len, group_roots, group_size, depth, slot0):
    """One extend batch: group g holds group_size tokens under root
    group_roots[g]; each token has `depth` private keys (fresh slots), the
    last its own."""
    G = len(group_roots)
    n = G * group_size
    ids = rng.integers(0, 1968, n).astype(np.int32)
    pos = np.full(n, prefix_len + depth - 1, np.int32)
    extra = (slot0 + np.arange(n * depth, dtype=np.int64)).reshape(n, depth).astype(np.int32)
    return dict(ids=ids, pos=pos, group_sizes=[group_size] * G,
                prefix_len=np.full(G, prefix_len, np.int32), prefix_blocks=table[list(group_roots)],
                extra_slot=extra, n_extra=np.full(n, depth, np.int32))


def run_both(eng, pool, b):
    st = torch.zeros(2, dtype=torch.int32, device=eng.device)
    ref = eng.extend(**b, kv_pool=pool, status=st[0:1])
    got = eng.extend(**b, kv_pool=pool, status=st[1:2], noalloc=True)
    torch.cuda.synchronize()
    assert st.tolist() == [0, 0]
    for f in FIELDS:
        a, c = getattr(ref, f), getattr(got, f)
        assert torch.equal(a, c), (f, (a != c).sum().item())
    return got


@pytest.mark.parametrize("mode", ["bfloat16", "fp8w", "float32"])
def test_noalloc_equals_extend_tiny(mode, cuda):
    cfg = config.TINY
    eng = Engine(cfg, weights.init_weights(cfg, seed=5, perturb=True), mode=mode)
    pool, table, free = roots(eng, 4, 37, seed=1)
    rng = np.random.default_rng(2)
    slot0 = free * 16
    # call 1: 4 groups of 5 children (fan kernel), 2 private keys each
    b1 = batch(rng, table, 37, [0, 1, 2, 3], 5, 2, slot0)
    r1 = run_both(eng, pool, b1)
    assert torch.isfinite(r1.logits).all()
    # call 2, smaller: 2 one-token groups (decode kernel), 3 private keys each
    b2 = batch(rng, table, 37, [3, 1], 1, 3, slot0 + 40)
    run_both(eng, pool, b2)
    eng.close()


def test_noalloc_medium_max_tokens(cuda):
    cfg = config.MEDIUM
    eng = Engine(cfg, weights.init_weights(cfg, seed=0), mode="bfloat16")
    pool, table, free = roots(eng, 4, 200, seed=3)
    rng = np.random.default_rng(4)
    slot0 = free * 16
    b1 = batch(rng, table, 200, [g % 4 for g in range(16)], 16, 1, slot0)  # 256 tokens
    run_both(eng, pool, b1)
    b2 = batch(rng, table, 200, [2, 0, 1], 1, 2, slot0 + 300)  # 3 tokens
    run_both(eng, pool, b2)
    b3 = batch(rng, table, 200, [g % 4 for g in range(257)], 1, 1, slot0)  # one token over the maximum
    with pytest.raises(capi.AllieError, match="max 256"):
        eng.extend(**b3, kv_pool=pool, noalloc=True)
    eng.close()


def test_noalloc_2x_fp8_max_tokens(cuda):
    cfg = config.LARGE2X
    eng = Engine(cfg, weights.init_weights(cfg, seed=0), mode="fp8w")
    pool, table, free = roots(eng, 4, 200, seed=3)
    rng = np.random.default_rng(6)
    slot0 = free * 16
    b1 = batch(rng, table, 200, [g % 4 for g in range(16)], 16, 1, slot0)  # 256 tokens
    run_both(eng, pool, b1)
    b2 = batch(rng, table, 200, [1, 3], 1, 2, slot0 + 300)
    run_both(eng, pool, b2)
    eng.close()


def test_noalloc_captured_with_allocation_forbidden(cuda):
    """The allocation-free extend captured into a HIP graph in the strictest
    capture mode (``global``: an allocation or free call from any thread
    during the capture fails it), then replayed three times with the
    allocating ``allie_extend`` run eagerly in between, each replay equal to
    it bit for bit; torch's allocator reserves nothing more across an eager
    call either."""
    from allie_amd.engine import PrefillResult

    cfg = config.TINY
    eng = Engine(cfg, weights.init_weights(cfg, seed=5, perturb=True), mode="bfloat16")
    pool, table, free = roots(eng, 4, 37, seed=1)
    rng = np.random.default_rng(8)
    b = batch(rng, table, 37, [0, 1, 2, 3, 2], 5, 2, free * 16)  # 25 tokens, fan kernel
    dev = eng.device
    n, G = len(b["ids"]), len(b["group_sizes"])
    gs = np.zeros(G + 1, np.int32)
    gs[1:] = np.cumsum(b["group_sizes"])
    i32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)
    ids, pos, gsd, pl = i32(b["ids"]), i32(b["pos"]), i32(gs), i32(b["prefix_len"])
    pb = b["prefix_blocks"].to(dtype=torch.int32).contiguous()
    ex, ne = i32(b["extra_slot"]), i32(b["n_extra"])
    V = cfg.vocab_size
    out = PrefillResult(logits=torch.zeros(n, V, device=dev), value=torch.zeros(n, device=dev),
                        time=torch.zeros(n, device=dev), top1=torch.zeros(n, dtype=torch.int32, device=dev),
                        max_logit=torch.zeros(n, device=dev), lse=torch.zeros(n, device=dev))
    status = torch.zeros(1, dtype=torch.int32, device=dev)

    def launch():
        eng.extend_noalloc_raw(ids, pos, gs, gsd, pl, pb, ex, ne, pool, out, status)

    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        launch()  # warm-up
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    before = (torch.cuda.memory_allocated(dev), torch.cuda.memory_reserved(dev))
    launch()
    torch.cuda.synchronize()
    assert (torch.cuda.memory_allocated(dev), torch.cuda.memory_reserved(dev)) == before
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, capture_error_mode="global"):
        launch()
    for rep in range(3):
        for f in FIELDS:
            getattr(out, f).zero_()
        status.fill_(-1)
        g.replay()
        ref = eng.extend(**b, kv_pool=pool)  # eager, allocating, between the replays
        torch.cuda.synchronize()
        assert int(status.item()) == 0, rep
        for f in FIELDS:
            assert torch.equal(getattr(out, f), getattr(ref, f)), (rep, f)
    eng.close()
