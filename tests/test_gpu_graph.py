"""HIP-graph capture of the library's entry points.  The library allocates,
frees and synchronises nothing, so a caller can capture a forward, a
backward or an index-producer call in a graph (the output and workspace
tensors come from the graph's memory pool).  Each test captures one call,
then replays it several times with eager work and synchronisations between
the replays and new input values written in place before each replay, and
checks every replay bitwise against an eager call on the same inputs (all
kernels on these paths are deterministic)."""
import sys

import pytest
import torch

import ops_amd

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _say(msg):
    print(f"\n[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        res = fn()
    torch.cuda.synchronize()
    return g, res


def _eager_noise(seed):
    # unrelated eager work between replays (library reductions included)
    x = torch.randn(1 << 20, device=DEV, generator=torch.Generator(device=DEV).manual_seed(seed))
    float(x.sum())
    torch.cuda.synchronize()


def _idx_rows(B, Sq, Hkv, K, hi_of_t, gen):
    idx = torch.full((B, Sq, Hkv, K), -1, dtype=torch.int32)
    for b in range(B):
        for t in range(Sq):
            hi = hi_of_t(b, t)
            n = min(K, hi)
            for h in range(Hkv):
                idx[b, t, h, :n] = torch.randperm(hi, generator=gen)[:n].to(torch.int32)
    return idx


def test_graph_mla_decode_splitk():
    """MLA decode (d_qk 576, d_v 512 = the first 512 dims of the K rows, 128
    heads) with 4 forced key splits: main kernel + combine kernel in one graph."""
    B, Skv, Hq, K = 4, 4096, 128, 1024
    _say(f"graph: MLA decode split-k B={B} Skv={Skv} Hq={Hq} K={K}")
    gen = torch.Generator().manual_seed(11)
    kv = torch.randn(B, Skv, 1, 576, generator=gen).to(torch.bfloat16).to(DEV)
    kv_lens = torch.tensor([4096, 3000, 1025, 2048], dtype=torch.int32, device=DEV)
    idx = _idx_rows(B, 1, 1, K, lambda b, t: int(kv_lens[b]), gen).to(DEV)
    sink = torch.randn(Hq, generator=gen).to(DEV)
    q = torch.empty(B, 1, Hq, 576, dtype=torch.bfloat16, device=DEV)
    v = kv[..., :512]

    def step():
        return ops_amd.sfa_forward(q, kv, v, idx, None, kv_lens=kv_lens, attn_sink=sink, num_splits=4)

    q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16))
    g, (out_g, lse_g) = _capture(step)
    for r in range(4):
        q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16))
        out_e, lse_e = step()
        torch.cuda.synchronize()
        _eager_noise(r)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {r}: out differs"
        assert torch.equal(lse_g, lse_e), f"replay {r}: lse differs"


def test_graph_mla_prefill_persistent_sorted():
    """Persistent MLA prefill (4160 work items, 128 heads on one latent row,
    d_qk 576 / d_v 512) on shuffled index rows: the index sort pass, the
    claim-counter reset and the persistent forward in one graph; new index
    rows and Q values are written in place before each replay, so every
    replay sorts and claims afresh."""
    S, K = 4160, 256
    _say(f"graph: persistent MLA prefill with the index sort pass S={S} K={K}")
    gen = torch.Generator().manual_seed(23)
    kv = torch.randn(1, S, 1, 576, generator=gen).to(torch.bfloat16).to(DEV)
    q = torch.empty(1, S, 128, 576, dtype=torch.bfloat16, device=DEV)
    idx = torch.empty(1, S, 1, K, dtype=torch.int32, device=DEV)
    v = kv[..., :512]

    def step():
        return ops_amd.sfa_forward(q, kv, v, idx, None)

    def refill():
        q.copy_(torch.randn(q.shape, generator=gen).to(torch.bfloat16))
        idx.copy_(_idx_rows(1, S, 1, K, lambda b, t: t + 1, gen))

    refill()
    g, (out_g, lse_g) = _capture(step)
    for r in range(3):
        refill()
        out_e, lse_e = step()
        torch.cuda.synchronize()
        _eager_noise(r)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), f"replay {r}: out differs"
        assert torch.equal(lse_g, lse_e), f"replay {r}: lse differs"


def test_graph_gqa_backward_deterministic():
    """GQA backward, deterministic dK/dV scheme: δ pass, index inversion, dQ,
    key-major dK/dV, chunk-ordered reduction and the bf16 finish in one graph."""
    B, S, Hq, Hkv, K = 1, 512, 32, 2, 256
    _say(f"graph: GQA backward (csr) B={B} S={S} Hq={Hq} Hkv={Hkv} K={K}")
    gen = torch.Generator().manual_seed(12)
    q = torch.randn(B, S, Hq, 128, generator=gen).to(torch.bfloat16).to(DEV)
    k = torch.randn(B, S, Hkv, 128, generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn(B, S, Hkv, 128, generator=gen).to(torch.bfloat16).to(DEV)
    idx = _idx_rows(B, S, Hkv, K, lambda b, t: t + 1, gen).to(DEV)
    out, lse = ops_amd.sfa_forward(q, k, v, idx)
    dout = torch.empty(B, S, Hq, 128, dtype=torch.bfloat16, device=DEV)

    def step():
        return ops_amd.sfa_backward(q, k, v, idx, out, lse, dout, dkv_mode="csr")[:3]

    dout.copy_(torch.randn(dout.shape, generator=gen).to(torch.bfloat16))
    g, grads_g = _capture(step)
    for r in range(4):
        dout.copy_(torch.randn(dout.shape, generator=gen).to(torch.bfloat16))
        grads_e = step()
        torch.cuda.synchronize()
        _eager_noise(r)
        g.replay()
        torch.cuda.synchronize()
        for name, a, e in zip(("dq", "dk", "dv"), grads_g, grads_e):
            assert torch.equal(a, e), f"replay {r}: {name} differs"


def test_graph_mla_backward_deterministic_three_chunks():
    """MLA shared-KV backward, deterministic: 2304 work items run as three
    chunks (1024, 1024, 256), so the graph holds the fork of each chunk's
    ordered reduction onto the library's second stream, chunk 2's index maps
    built there after chunk 0's reduction (the buffer set they share), the
    wait of chunk 2's dK/dV pass for them, and the join before the sink
    gradient and the finish."""
    B, S, Hq, K = 1, 2304, 128, 256
    _say(f"graph: MLA backward (deterministic) B={B} S={S} Hq={Hq} K={K}, three chunks")
    gen = torch.Generator().manual_seed(21)
    q = torch.randn(B, S, Hq, 576, generator=gen).to(torch.bfloat16).to(DEV)
    kv = torch.randn(B, S, 1, 576, generator=gen).to(torch.bfloat16).to(DEV)
    idx = _idx_rows(B, S, 1, K, lambda b, t: t + 1, gen).to(DEV)
    sink = torch.linspace(-1.0, 1.0, Hq).to(DEV)
    scale = 576 ** -0.5
    out, lse = ops_amd.sfa_forward(q, kv, kv[..., :512], idx, scale, attn_sink=sink)
    dout = torch.empty(B, S, Hq, 512, dtype=torch.bfloat16, device=DEV)

    def step():
        return ops_amd.sfa_backward(q, kv, kv[..., :512], idx, out, lse, dout, scale, attn_sink=sink,
                                    merge_kv=True, dkv_mode="csr")

    dout.copy_(torch.randn(dout.shape, generator=gen).to(torch.bfloat16))
    g, grads_g = _capture(step)
    for r in range(4):
        dout.copy_(torch.randn(dout.shape, generator=gen).to(torch.bfloat16))
        grads_e = step()
        torch.cuda.synchronize()
        _eager_noise(r)
        g.replay()
        torch.cuda.synchronize()
        for name, a, e in zip(("dq", "dkv", "dsink"), (grads_g[0], grads_g[1], grads_g[3]),
                              (grads_e[0], grads_e[1], grads_e[3])):
            assert torch.equal(a, e), f"replay {r}: {name} differs"


def test_graph_indexer_topk():
    """Index producer (scores kernel + selection kernel per query chunk)."""
    B, S, H, topk = 1, 1024, 64, 256
    _say(f"graph: indexer B={B} S={S} H={H} topk={topk}")
    gen = torch.Generator().manual_seed(13)
    qi = torch.empty(B, S, H, 128, dtype=torch.bfloat16, device=DEV)
    ki = torch.randn(B, S, 128, generator=gen).to(torch.bfloat16).to(DEV)
    w = torch.rand(B, S, H, generator=gen).to(DEV) * 0.1

    def step():
        return ops_amd.indexer_topk(qi, ki, w, topk)

    qi.copy_(torch.randn(qi.shape, generator=gen).to(torch.bfloat16))
    g, idx_g = _capture(step)
    for r in range(3):
        qi.copy_(torch.randn(qi.shape, generator=gen).to(torch.bfloat16))
        idx_e = step()
        torch.cuda.synchronize()
        _eager_noise(r)
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(idx_g, idx_e), f"replay {r}: indices differ"
