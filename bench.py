"""Verify-step benchmark on one MI355X: packed-window paged attention, target
distributions from logits, acceptance.

Workload (the verify-step config the metric is quoted on):
batch 32 requests x verify window q_len = k + 1 = 5 with the intra-window causal
mask; 16 q heads / 4 kv heads (GQA 4), head_dim 128, bf16 KV in the SHARED layout
(one plane), context lengths uniform in [1024, 8192]; block size 16, block tables a
seeded random permutation of the pool.  Acceptance over vocab 49152 with target /
draft distributions built at temperature 0.7, top-p 0.9, seeded per-request
uniforms.  Synthetic data, random values: there is no model or dataset.

One step = the KV write of the 160 window rows' keys and values into the pool (the
writer that precedes attention in every layer, vllm_rlt/kernels/graph_kv.py:52-67) +
the attention call over all 160 verify rows + the verify side of the round (the
argmax of every verify row and the distributions of the 160 target-logit rows, fp32,
T = 0.7, top-p 0.9: the reference's _verify, vllm_rlt/worker/async_speculative.py:678-692,
in one launch) + speculative_accept over the 32
requests (draft distributions q are inputs, made in the draft step); the verify side
and the acceptance run as one ``verify_accept`` call, whose distribution launch also
sums the draft rows for the acceptance.  All replayed
from HIP graphs (the reference runs its recurrent core under graphs too).
``value`` = verified tokens (32 x 5) / step time.

Output: one JSON line (see the driver contract) with ``roofline`` for the
attention launch (algorithmic bytes / average launch time, HIP events on the launch
stream) and ``cpu_baseline`` (the torch-CPU oracle on this host).
"""

import argparse
import hashlib
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "verified tokens/sec on 1 MI355X (verify attn+accept); % of HBM peak GB/s"


def probabilities(logits, temperature, top_p):
    """softmax(logits / T) restricted to the top-p nucleus (data generation only)."""
    x = logits.float() / temperature
    if top_p < 1:
        sx, idx = x.sort(dim=-1, descending=True)
        drop = sx.softmax(-1).cumsum(-1) > top_p
        drop[..., 1:] = drop[..., :-1].clone()
        drop[..., 0] = False
        x = x.scatter(-1, idx, sx.masked_fill(drop, -torch.inf))
    return x.softmax(-1)


def build_workload(dev, seed=0, n=32, ctx=None):
    """Config 3 (n = 32, ctx U[1024, 8192]); ``ctx`` fixes every context length instead."""
    window, hq, hkv, d, bs, layers, vocab = 5, 16, 4, 128, 16, 2, 49152
    k_drafts = window - 1
    g = torch.Generator().manual_seed(seed)
    lengths = torch.randint(1024, 8193, (n,), generator=g, dtype=torch.int64)
    if ctx is not None:
        lengths = torch.full((n,), ctx, dtype=torch.int64)
    width = 8192 // bs
    pool = n * width
    tables = torch.randperm(pool, generator=g)[: n * width].view(n, width).int()
    gd = torch.Generator(device=dev).manual_seed(seed)
    shape = (pool, layers, bs, hkv, d)
    key_pool = torch.randn(shape, generator=gd, device=dev, dtype=torch.bfloat16)
    value_pool = torch.randn(shape, generator=gd, device=dev, dtype=torch.bfloat16)
    q = torch.randn(n * window, hq, d, generator=gd, device=dev, dtype=torch.bfloat16)
    cu = torch.arange(0, n * window + 1, window, dtype=torch.int32)
    draft_logits = torch.randn(n, window, vocab, generator=gd, device=dev) * 3.0
    target_logits = draft_logits + torch.randn(n, window, vocab, generator=gd, device=dev)
    qprob = probabilities(draft_logits[:, :k_drafts], 0.7, 0.9).contiguous()
    pprob = probabilities(target_logits, 0.7, 0.9).contiguous()
    seeds = torch.randint(0, 2**31, (n,), generator=g).tolist()
    u = torch.stack([torch.rand(2 * k_drafts + 1, generator=torch.Generator().manual_seed(s))
                     for s in seeds])
    # the window's own keys / values and where they go: position len - window + j
    k_new = torch.randn(n * window, hkv, d, generator=gd, device=dev, dtype=torch.bfloat16)
    v_new = torch.randn(n * window, hkv, d, generator=gd, device=dev, dtype=torch.bfloat16)
    pos = (lengths.view(n, 1) - window + torch.arange(window).view(1, window)).reshape(-1)
    req = torch.arange(n).repeat_interleave(window)
    w_blocks = tables[req, pos // bs].long()
    w_offsets = pos % bs
    return dict(n=n, window=window, hq=hq, hkv=hkv, d=d, bs=bs, vocab=vocab, k=k_drafts,
                k_new=k_new, v_new=v_new, w_blocks=w_blocks.to(dev), w_offsets=w_offsets.to(dev),
                lengths=lengths, tables=tables, key_pool=key_pool, value_pool=value_pool, q=q,
                cu=cu, qprob=qprob, pprob=pprob, u=u, layer=1,
                target_logits=target_logits.reshape(n * window, vocab).contiguous(),
                temperature=0.7, top_p=0.9)


def attention_bytes(w):
    """Algorithmic HBM bytes of one attention launch: each needed KV byte once per
    (request, plane) up to the last window row, plus q, out and the table entries."""
    elt = 2
    kv = int(w["lengths"].sum()) * 2 * w["hkv"] * w["d"] * elt
    qo = 2 * w["n"] * w["window"] * w["hq"] * w["d"] * elt
    tables = int(sum(math.ceil(int(n) / w["bs"]) for n in w["lengths"])) * 4
    return kv + qo + tables


def kv_write_bytes(w):
    """Window K and V rows read once and written once (bf16), plus the int64 addresses."""
    rows = w["n"] * w["window"]
    return 2 * 2 * rows * w["hkv"] * w["d"] * 2 + 16 * rows


def probs_bytes(w):
    """fp32 target logits read once, fp32 distributions written once."""
    return 2 * 4 * w["n"] * w["window"] * w["vocab"] + 16 * w["n"] * w["window"]


def accept_bytes(w):
    n, k, v = w["n"], w["k"], w["vocab"]
    return 4 * n * (k + 1) * v + 4 * n * k * v + 4 * n * (2 * k + 1) + 8 * n * (k + 1) + 8 * n * 3 + 8 * n * k


def kernel_source_digest():
    """First 16 hex digits of a sha256 over the library's HIP sources and headers (names
    and contents, sorted by name): identifies the build a counter measurement is of."""
    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "vllm-rlt_amd", "csrc")
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def measured_traffic():
    """HBM bytes per attention launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (calibrated against a 1 GiB copy), and whether they were measured
    on the kernel sources of this tree: (bytes or None, record)."""
    path = os.path.join(ROOT, "profiles", "verify_step_config3_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None, {}
    same = rec.get("kernel_source_digest") == kernel_source_digest()
    return (rec.get("attention_launch_bytes") if same else None), rec


def config2_decode(pkg, dev):
    """BASELINE.json configs[1] (the decode attention config the >=70%-of-HBM target names:
    batch 64, ctx U[512, 4096]): one launch, its algorithmic bytes and bandwidth."""
    g = torch.Generator().manual_seed(2)
    n, planes, bs, h, d = 64, 4, 16, 16, 128
    lengths = torch.randint(512, 4097, (n,), generator=g)
    exit_depth = torch.randint(1, 5, (n,), generator=g)
    width = 4096 // bs
    pool = n * planes * width
    gd = torch.Generator(device=dev).manual_seed(2)
    k = torch.randn(pool, bs, h, d, generator=gd, device=dev, dtype=torch.bfloat16)
    v = torch.randn(pool, bs, h, d, generator=gd, device=dev, dtype=torch.bfloat16)
    tables = torch.randperm(pool, generator=g).int().view(n, planes, width)
    rows = tables[torch.arange(n), exit_depth - 1].to(dev)
    q = torch.randn(n, h, d, generator=gd, device=dev, dtype=torch.bfloat16)
    ctx = lengths.int().to(dev)
    kern = pkg.MI355XPagedAttention()
    t, _ = _graph_time(lambda: kern(q, k, v, rows, ctx))
    nbytes = int(lengths.sum()) * 2 * h * d * 2 + 2 * n * h * d * 2 + int(
        sum(math.ceil(int(x) / bs) for x in lengths)) * 4
    return {"workload": "config2 decode attention: batch 64, ctx U[512,4096], 16/16 heads, D=128, "
                        "bf16, 4 LAST_EXITED planes, exit depth U{1..4}",
            "us": round(t * 1e6, 1), "algorithmic_bytes": nbytes,
            "GBps": round(nbytes / t / 1e9, 1), "frac": round(nbytes / t / 1e9 / PEAK_HBM_GBS, 4)}


def _graph_time(fn, reps=21, per_graph=10):
    """Median launch time of ``fn`` over ``reps`` replays of a HIP graph of ``per_graph``
    calls, HIP events on the current stream, queue pre-filled."""
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(per_graph):
            out = fn()
    graph.replay()
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    torch.cuda._sleep(50_000_000)
    for a, b in ev:
        a.record(s)
        graph.replay()
        b.record(s)
    torch.cuda.synchronize()
    times = sorted(a.elapsed_time(b) for a, b in ev)
    t = times[len(times) // 2] / 1e3 / per_graph
    eager = fn()
    torch.cuda.synchronize()
    same = all(torch.equal(x, y) for x, y in zip(_flat(eager), _flat(out)))
    del graph
    return t, same


def _flat(x):
    if isinstance(x, torch.Tensor):
        return [x]
    out = []
    for y in x:
        out.extend(_flat(y))
    return out


def _fp8_pool(shape, dev, gd):
    """Random finite float8_e4m3fn bytes (0x7f / 0xff are NaN), filled in 1 GiB pieces."""
    buf = torch.empty(shape, dtype=torch.uint8, device=dev)
    flat = buf.view(-1)
    step = 1 << 30
    for i in range(0, flat.numel(), step):
        c = flat[i:i + step]
        c.random_(0, 255, generator=gd)
        c.masked_fill_(c == 0x7F, 0x7E)
    return buf.view(torch.float8_e4m3fn)


def _accept_part(pkg, dev, gd, n, window, vocab):
    """The verify round at T = 1, no truncation (configs 4 and 5 name no truncation):
    target argmax, distributions and acceptance in one ``verify_accept`` call."""
    k = window - 1
    draft_logits = torch.randn(n, k, vocab, generator=gd, device=dev) * 3.0
    target_logits = torch.cat([draft_logits, draft_logits[:, :1]], 1) + torch.randn(
        n, window, vocab, generator=gd, device=dev)
    qprob = draft_logits.softmax(-1).contiguous()
    u = torch.rand(n, 2 * k + 1, generator=gd, device=dev)
    drafts_tok = torch.stack([pkg.categorical(qprob[:, j].contiguous(), u[:, j].contiguous())[0]
                              for j in range(k)], 1)
    drafts = torch.full((n,), k, dtype=torch.int64, device=dev)
    rows = n * window
    temp = torch.ones(rows, device=dev)
    top_k = torch.full((rows,), -1, dtype=torch.int64, device=dev)
    top_p = torch.ones(rows, device=dev)
    ua, uf = u[:, k:2 * k].contiguous(), u[:, 2 * k].contiguous()

    def verify():
        return pkg.verify_accept(target_logits, temp, top_k, top_p, drafts_tok, drafts, qprob, ua, uf,
                                 max_top_k=0, apply_top_p=False)

    t, same = _graph_time(verify)
    nbytes = 2 * 4 * rows * vocab + 4 * n * k * vocab + 4 * n * (2 * k + 1) + 8 * n * (k + 1) + 8 * rows
    return t, same, nbytes


def _kv_bytes_distinct(tables, lengths, req_of_row, kv_heads, head_dim, elt, bs):
    """Each needed KV byte once per (request, block table): the longest row reading it."""
    longest = {}
    for r in range(tables.shape[0]):
        key = (int(req_of_row[r]), tuple(tables[r, :4].tolist()))
        longest[key] = max(longest.get(key, 0), int(lengths[r]))
    toks = sum(longest.values())
    return toks * 2 * kv_heads * head_dim * elt + sum(-(-x // bs) for x in longest.values()) * 4


def config4_step(pkg, dev):
    """55 q / kv heads, head_dim 96, 32 LAST_EXITED planes with exit
    depth U{8..32}, batch 16, ctx 2048, verify window 5 (packed form), acceptance at V = 65536."""
    g = torch.Generator().manual_seed(4)
    gd = torch.Generator(device=dev).manual_seed(4)
    n, w, planes, bs, h, d, ctx_len, vocab = 16, 5, 32, 16, 55, 96, 2048, 65536
    per = ctx_len // bs
    pool = n * planes * per
    k = torch.randn(pool, bs, h, d, generator=gd, device=dev, dtype=torch.bfloat16)
    v = torch.randn(pool, bs, h, d, generator=gd, device=dev, dtype=torch.bfloat16)
    tables = torch.randperm(pool, generator=g).int().view(n, planes, per)
    exit_depth = torch.randint(8, 33, (n,), generator=g)
    seq_tables = tables[torch.arange(n), exit_depth - 1].to(dev)
    lengths = torch.full((n,), ctx_len, dtype=torch.int32, device=dev)
    q = torch.randn(n * w, h, d, generator=gd, device=dev, dtype=torch.bfloat16)
    cu = torch.arange(0, n * w + 1, w, dtype=torch.int32, device=dev)
    kern = pkg.MI355XPagedAttention()
    t_attn, same_attn = _graph_time(lambda: kern.prefill(q, k, v, seq_tables, lengths, cu, w))
    a_bytes = n * ctx_len * 2 * h * d * 2 + 2 * n * w * h * d * 2 + n * per * 4
    del k, v
    t_acc, same_acc, c_bytes = _accept_part(pkg, dev, gd, n, w, vocab)
    return _secondary("config4: 55/55 heads, D=96, bf16, 32 LAST_EXITED planes (exit depth U{8..32}), "
                      "batch 16, ctx 2048, packed q_len=5; verify_accept V=65536, T=1, no truncation",
                      n * w, t_attn, a_bytes, t_acc, c_bytes, same_attn and same_acc)


def config5_step(pkg, dev, attention_only=False):
    """fp8-e4m3 KV with per-tensor fp32 scales, batch 256, ctx
    U[16384, 32768], q_len 5 with window row j at plane (d0 + j) mod 4, 16 q / 8 kv heads,
    D = 128; acceptance at V = 65536.  Attention is timed twice: the reference's per-row form
    (one gathered table and length per row) and one packed sequence per (request, plane) with
    explicit row lengths (bitwise the same rows; the plane rows 0 and 4 share is read once)."""
    g = torch.Generator().manual_seed(5)
    gd = torch.Generator(device=dev).manual_seed(5)
    n, w, planes, bs, hq, hkv, d, vocab = 256, 5, 4, 16, 16, 8, 128, 65536
    max_len = 32768 + w
    per = -(-max_len // bs)
    pool = n * planes * per
    kc = _fp8_pool((pool, bs, hkv, d), dev, gd)
    vc = _fp8_pool((pool, bs, hkv, d), dev, gd)
    tables = torch.randperm(pool, generator=g).int().view(n, planes, per)
    start = torch.randint(16384 - w, 32768 - w + 1, (n,), generator=g)
    d0 = torch.randint(0, planes, (n,), generator=g)
    j = torch.arange(w)
    plane = (d0.view(n, 1) + j.view(1, w)) % planes
    row_tables = tables[torch.arange(n).view(n, 1), plane].reshape(n * w, per)
    row_len = (start.view(n, 1) + j.view(1, w) + 1).reshape(-1).int()
    req = torch.arange(n).repeat_interleave(w)
    q = torch.randn(n * w, hq, d, generator=gd, device=dev, dtype=torch.bfloat16)
    sk = torch.tensor(0.03, device=dev)
    sv = torch.tensor(0.05, device=dev)
    rt, rl = row_tables.to(dev), row_len.to(dev)
    kern = pkg.MI355XPagedAttention()
    # the same rows as one packed sequence per (request, plane) with explicit row lengths:
    # rows j = 0 and j = 4 read plane d0 once between them
    perm, cu = [], [0]
    seq_tables, seq_len = [], []
    for i in range(n):
        for pl in range(planes):
            rows = [i * w + jj for jj in range(w) if int(plane[i, jj]) == pl]
            if rows:
                perm += rows
                cu.append(len(perm))
                seq_tables.append(tables[i, pl])
                seq_len.append(int(row_len[rows[-1]]))
    perm_d = torch.tensor(perm, device=dev)
    st, sl = torch.stack(seq_tables).to(dev), torch.tensor(seq_len, dtype=torch.int32, device=dev)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=dev)
    max_q = max(cu[s + 1] - cu[s] for s in range(len(cu) - 1))
    qp, rlp = q[perm_d].contiguous(), row_len.to(dev)[perm_d].contiguous()
    if attention_only:  # counter collection: two per-row launches, then two packed launches
        for _ in range(2):
            kern(q, kc, vc, rt, rl, sk, sv)
        for _ in range(2):
            kern.prefill(qp, kc, vc, st, sl, cu_d, max_q, sk, sv, row_lengths=rlp)
        torch.cuda.synchronize()
        return {"only": "config5_attention", "launches": 4}
    t_row, same_row = _graph_time(lambda: kern(q, kc, vc, rt, rl, sk, sv), reps=5, per_graph=4)
    t_attn, same_attn = _graph_time(
        lambda: kern.prefill(qp, kc, vc, st, sl, cu_d, max_q, sk, sv, row_lengths=rlp),
        reps=5, per_graph=4)
    packed_equal = torch.equal(kern.prefill(qp, kc, vc, st, sl, cu_d, max_q, sk, sv, row_lengths=rlp),
                               kern(q, kc, vc, rt, rl, sk, sv)[perm_d])
    # the window's own K / V quantized into the pool by the attention launch (each row at
    # position row_lengths - 1 of its plane), against store_fp8 then the same attention;
    # replays rewrite the same codes.  One fixed scale for K and V here (store_fp8 takes one)
    kn = (torch.randn(n * w, hkv, d, generator=gd, device=dev) * 2).bfloat16()[perm_d].contiguous()
    vn = (torch.randn(n * w, hkv, d, generator=gd, device=dev) * 2).bfloat16()[perm_d].contiguous()
    seq_of_row = torch.repeat_interleave(torch.arange(len(cu) - 1), torch.tensor(cu[1:]) - torch.tensor(cu[:-1]))
    pos = row_len[torch.tensor(perm)].long() - 1
    w_blocks = torch.stack(seq_tables).long()[seq_of_row, pos // bs].to(dev)
    w_offs = (pos % bs).to(dev)
    sp = torch.zeros(n * w, device=dev)  # scratch scale rows for store_fp8 (fixed scale)
    sp_pool = sp.new_zeros(())  # not read with a fixed scale
    scratch_scales = torch.zeros(pool, bs, hkv, device=dev)

    def separate():
        pkg.store_fp8(kn, vn, kc, vc, scratch_scales, scratch_scales, w_blocks, w_offs, 448.0,
                      fixed_scale=0.03)
        return kern.prefill(qp, kc, vc, st, sl, cu_d, max_q, sk, sk, row_lengths=rlp)

    fused = lambda: kern.prefill_store(qp, kn, vn, kc, vc, st, sl, cu_d, max_q, sk, sk,  # noqa: E731
                                       row_lengths=rlp)
    store_equal = torch.equal(separate(), fused())
    t_store_only, _ = _graph_time(
        lambda: (pkg.store_fp8(kn, vn, kc, vc, scratch_scales, scratch_scales, w_blocks, w_offs,
                               448.0, fixed_scale=0.03), kc)[1], reps=5, per_graph=4)
    t_fused, same_fused = _graph_time(fused, reps=5, per_graph=4)
    del sp, sp_pool, scratch_scales
    a_bytes = _kv_bytes_distinct(row_tables, row_len, req, hkv, d, 1, bs) + 2 * n * w * hq * d * 2
    row_bytes = int(row_len.sum()) * 2 * hkv * d
    del kc, vc
    t_acc, same_acc, c_bytes = _accept_part(pkg, dev, gd, n, w, vocab)
    out = _secondary("config5: fp8-e4m3 KV, per-tensor scales, batch 256, ctx U[16384,32768], 16/8 heads, "
                     "D=128, window row j at plane (d0+j) mod 4, packed per (request, plane) with "
                     "row_lengths; verify_accept V=65536, T=1, no truncation", n * w, t_attn, a_bytes,
                     t_acc, c_bytes, same_attn and same_acc and same_row)
    out["packed_rows_equal_per_row_bitwise"] = packed_equal
    out["attention_with_kv_store_us"] = round(t_fused * 1e6, 1)
    out["kv_store_fp8_us"] = round(t_store_only * 1e6, 1)
    out["kv_store_fused_equals_store_fp8_then_attention"] = store_equal and same_fused
    out["per_row_attention_us"] = round(t_row * 1e6, 1)
    out["per_row_attention_frac"] = round(a_bytes / t_row / 1e9 / PEAK_HBM_GBS, 4)
    out["per_row_read_GBps"] = round(row_bytes / t_row / 1e9, 1)
    return out



def target_step(pkg, dev):
    """The shape the north-star target names: the verify step at batch 64, ctx 4096 (config 3's
    heads, window and sampling otherwise).  Reports attention + speculative_accept (the
    acceptance from p and q, the bit-exact contract) and attention + verify_accept (the
    distributions from logits too), each as algorithmic bytes over summed launch times."""
    w = build_workload(dev, seed=7, n=64, ctx=4096)
    k = w["k"]
    kc, vc = w["key_pool"][:, w["layer"]], w["value_pool"][:, w["layer"]]
    tables, lengths, cu = w["tables"].to(dev), w["lengths"].int().to(dev), w["cu"].to(dev)
    u = w["u"].to(dev)
    ua, uf = u[:, k:2 * k].contiguous(), u[:, 2 * k].contiguous()
    drafts = torch.full((w["n"],), k, dtype=torch.int64, device=dev)
    dt_tok = torch.stack([pkg.categorical(w["qprob"][:, j].contiguous(), u[:, j].contiguous())[0]
                          for j in range(k)], 1)
    rows = w["n"] * w["window"]
    temp = torch.full((rows,), w["temperature"], device=dev)
    top_k = torch.full((rows,), -1, dtype=torch.int64, device=dev)
    top_p = torch.full((rows,), w["top_p"], device=dev)
    kern = pkg.MI355XPagedAttention()
    logits3 = w["target_logits"].view(w["n"], w["window"], -1)
    t_attn, s1 = _graph_time(lambda: kern.prefill(w["q"], kc, vc, tables, lengths, cu, w["window"]))
    t_acc, s2 = _graph_time(lambda: pkg.speculative_accept(dt_tok, drafts, w["qprob"], w["pprob"], ua, uf))
    t_ver, s3 = _graph_time(lambda: pkg.verify_accept(logits3, temp, top_k, top_p, dt_tok, drafts,
                                                      w["qprob"], ua, uf, max_top_k=0,
                                                      apply_top_p=True))
    a, c, pb = attention_bytes(w), accept_bytes(w), probs_bytes(w)
    frac = lambda b, t: round(b / t / 1e9 / PEAK_HBM_GBS, 4)
    return {"workload": "verify step at batch 64, ctx 4096: packed q_len=5, 16q/4kv heads, D=128, bf16 "
                        "SHARED KV; acceptance V=49152, T=0.7, top-p 0.9",
            "attention_us": round(t_attn * 1e6, 1), "attention_algorithmic_bytes": a,
            "attention_frac": frac(a, t_attn),
            "accept_us": round(t_acc * 1e6, 1), "accept_algorithmic_bytes": c,
            "attention_plus_accept_frac": frac(a + c, t_attn + t_acc),
            "verify_accept_us": round(t_ver * 1e6, 1),
            "attention_plus_verify_accept_frac": frac(a + c + pb, t_attn + t_ver),
            "verified_tokens_per_s": round(rows / (t_attn + t_ver), 1),
            "graph_replays_equal_eager": s1 and s2 and s3}

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def draft_steps(pkg, dev):
    """One draft offset of the _draft step (async_speculative.py:645-663): argmax of every
    row, the random rows' distributions q_o and their categorical draws, in one
    ``propose_drafts`` call.  Config 3's shape (32 requests, V = 49152, T = 0.7, top-p 0.9:
    the filtered single-workgroup form) and config 5's (256 requests, V = 65536, T = 1, no
    truncation: the row-split form).  Algorithmic bytes: the fp32 logits read once and q_o
    written once."""
    g = torch.Generator(device=dev).manual_seed(7)
    out = {}
    for name, m, vocab, temp, top_p in (("config3", 32, 49152, 0.7, 0.9),
                                        ("config5", 256, 65536, 1.0, 1.0)):
        logits = torch.randn(m, vocab, generator=g, device=dev) * 4
        rows = torch.arange(m, device=dev)
        t = torch.full((m,), temp, device=dev)
        tk = torch.full((m,), -1, dtype=torch.int64, device=dev)
        tp = torch.full((m,), top_p, device=dev)
        u = torch.rand(m, generator=g, device=dev)
        filt = top_p < 1.0
        t_us, same = _graph_time(lambda: pkg.propose_drafts(logits, rows, t, tk, tp, u, max_top_k=0,
                                                            apply_top_p=filt))
        nbytes = 2 * 4 * m * vocab
        out[name] = {"rows": m, "vocab": vocab, "us": round(t_us * 1e6, 1),
                     "algorithmic_bytes": nbytes,
                     "frac_hbm": round(nbytes / t_us / 1e9 / PEAK_HBM_GBS, 4),
                     "graph_replays_equal_eager": same}
        del logits
    return {"workload": "one draft offset: argmax + distributions + categorical draws "
                        "(propose_drafts), all rows random", "launches": out}


def prefill_steps(pkg, dev):
    """The packed causal prefill tiling (a prompt's whole window attends to itself through the
    pool, triton_attention.py:250-383): bf16, 16 q / 4 kv heads, D = 128, block size 16; batches
    of 8 x 2048, 4 x 4096 and 1 x 8192-token prompts.  MFMA-bound: 4 * Hq * D * sum L(L+1)/2
    flops per launch."""
    g = torch.Generator().manual_seed(6)
    gd = torch.Generator(device=dev).manual_seed(6)
    hq, hkv, d, bs = 16, 4, 128, 16
    kern = pkg.MI355XPagedAttention()
    out = {}
    for n, L in ((8, 2048), (4, 4096), (1, 8192)):
        per = L // bs
        kc = torch.randn(n * per, bs, hkv, d, generator=gd, device=dev, dtype=torch.bfloat16)
        vc = torch.randn(n * per, bs, hkv, d, generator=gd, device=dev, dtype=torch.bfloat16)
        tables = torch.randperm(n * per, generator=g).int().view(n, per).to(dev)
        lengths = torch.full((n,), L, dtype=torch.int32, device=dev)
        cu = torch.arange(0, n * L + 1, L, dtype=torch.int32, device=dev)
        q = torch.randn(n * L, hq, d, generator=gd, device=dev, dtype=torch.bfloat16)
        t, same = _graph_time(lambda: kern.prefill(q, kc, vc, tables, lengths, cu, L), reps=11,
                              per_graph=4)
        flops = 4 * hq * d * n * L * (L + 1) // 2
        tf = flops / t / 1e12
        out[f"{n}x{L}"] = {"us": round(t * 1e6, 1), "tflops": round(tf, 1),
                           "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                           "graph_replays_equal_eager": same}
        del kc, vc, q
    # fp8 pools (the verify kernel's packed form at prompt length) and head_dim 96 (the
    # prefill tiling on 128-dim LDS rows)
    n, L = 8, 2048
    per = L // bs
    tables = torch.randperm(n * per, generator=g).int().view(n, per).to(dev)
    lengths = torch.full((n,), L, dtype=torch.int32, device=dev)
    cu = torch.arange(0, n * L + 1, L, dtype=torch.int32, device=dev)
    for name, dd, kv_dtype in (("fp8_d128_8x2048", 128, torch.float8_e4m3fn),
                               ("bf16_d96_8x2048", 96, torch.bfloat16)):
        if kv_dtype == torch.float8_e4m3fn:
            kc = _fp8_pool((n * per, bs, hkv, dd), dev, gd)
            vc = _fp8_pool((n * per, bs, hkv, dd), dev, gd)
            scales = (torch.tensor(0.03, device=dev), torch.tensor(0.05, device=dev))
        else:
            kc = torch.randn(n * per, bs, hkv, dd, generator=gd, device=dev, dtype=kv_dtype)
            vc = torch.randn(n * per, bs, hkv, dd, generator=gd, device=dev, dtype=kv_dtype)
            scales = (None, None)
        q = torch.randn(n * L, hq, dd, generator=gd, device=dev, dtype=torch.bfloat16)
        t, same = _graph_time(lambda: kern.prefill(q, kc, vc, tables, lengths, cu, L, *scales),
                              reps=5, per_graph=2)
        flops = 4 * hq * dd * n * L * (L + 1) // 2
        tf = flops / t / 1e12
        out[name] = {"us": round(t * 1e6, 1), "tflops": round(tf, 1),
                     "frac_bf16_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                     "path": ("prefill tiling" if kern.uses_prefill_tiling(
                         torch.bfloat16, kv_dtype, dd, L) else "verify kernel, packed form"),
                     "graph_replays_equal_eager": same}
        del kc, vc, q
    return {"workload": "packed causal prefill, bf16, 16 q / 4 kv heads, D=128, block 16 (the "
                        "prefill tiling); fp8-e4m3 (per-tensor scales) and D=96 prompts as "
                        "labelled by each entry's path",
            "flops_per_launch": "4 * Hq * D * sum L(L+1)/2", "launches": out}


def _secondary(workload, tokens, t_attn, a_bytes, t_acc, c_bytes, replay_equal):
    return {"workload": workload,
            "verified_tokens_per_s": round(tokens / (t_attn + t_acc), 1),
            "attention_us": round(t_attn * 1e6, 1), "attention_algorithmic_bytes": a_bytes,
            "attention_GBps": round(a_bytes / t_attn / 1e9, 1),
            "attention_frac": round(a_bytes / t_attn / 1e9 / PEAK_HBM_GBS, 4),
            "verify_accept_us": round(t_acc * 1e6, 1), "verify_accept_algorithmic_bytes": c_bytes,
            "verify_accept_GBps": round(c_bytes / t_acc / 1e9, 1),
            "graph_replays_equal_eager": replay_equal}


def cpu_baseline(w, repeats=1):
    """The torch-CPU oracle (restatement of the reference Torch path) on this host."""
    from oracle import attention as oatt
    from oracle import kv_write as okv
    from oracle import sampling as osamp

    k_view = w["key_pool"][:, w["layer"]].cpu()
    v_view = w["value_pool"][:, w["layer"]].cpu()
    q, tables, lengths, cu = w["q"].cpu(), w["tables"], w["lengths"].int(), w["cu"]
    qprob, u = w["qprob"].cpu(), w["u"]
    logits = w["target_logits"].cpu()
    rows = logits.shape[0]
    temp = torch.full((rows,), w["temperature"])
    top_k = torch.full((rows,), -1, dtype=torch.int64)
    top_p = torch.full((rows,), w["top_p"])
    drafts_tok = w["draft_tokens"].cpu()
    drafts = torch.full((w["n"],), w["k"], dtype=torch.int64)
    k = w["k"]
    k_new, v_new = w["k_new"].cpu(), w["v_new"].cpu()
    w_blocks, w_offsets = w["w_blocks"].cpu(), w["w_offsets"].cpu()
    t0 = time.perf_counter()
    for _ in range(repeats):
        okv.store_kv(k_view, v_view, k_new, v_new, w_blocks, w_offsets)
        oatt.packed_window_attention(q, k_view, v_view, tables, lengths, cu)
        pprob = osamp.batched_probabilities(logits, temp, top_k, top_p, max_top_k=0,
                                            apply_top_p=True).view(w["n"], w["window"], -1)
        osamp.speculative_accept(drafts_tok, drafts, qprob, pprob, u[:, k:2 * k].contiguous(),
                                 u[:, 2 * k].contiguous())
    dt = (time.perf_counter() - t0) / repeats
    return {"value": round(w["n"] * w["window"] / dt, 2), "unit": "verified tokens/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"full config3 verify step (window KV write, 32 requests x 5 rows, ctx U[1024,8192]) x {repeats}, "
                      f"{dt * 1e3:.0f} ms per step, torch-CPU oracle "
                      f"(os.cpu_count={os.cpu_count()})"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-config2", action="store_true",
                    help="skip the secondary config-2 decode attention measurement")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the config-4 and config-5 attention + verify_accept measurements")
    ap.add_argument("--prefill-only", action="store_true",
                    help="print only the prefill measurements and exit")
    ap.add_argument("--draft-only", action="store_true",
                    help="print only the draft-step measurements and exit")
    ap.add_argument("--only", choices=("kv_write", "attention", "attention_store", "probs", "accept",
                                       "verify", "copy",
                                       "config5_attention"),
                    help="replay only this part K times and exit (for counter collection); "
                         "'copy' copies a 1 GiB buffer K times (counter calibration); "
                         "'config5_attention' runs the config-5 attention twice per-row, then "
                         "twice packed with row lengths")
    ap.add_argument("--steps-per-graph", type=int, default=10,
                    help="verify steps captured back to back in one HIP graph")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only: the verify path has no "
                                   "cross-GPU exchange (requests shard by data parallelism); "
                                   "run with --gpus 1"}))
        sys.exit(2)
    pkg = __graft_entry__.load_package()
    dev = torch.device("cuda:0")
    if args.only == "copy":
        src_buf = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
        dst_buf = torch.empty_like(src_buf)
        for _ in range(args.steps):
            dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        print(json.dumps({"only": "copy", "bytes_per_launch": 1 << 30, "steps": args.steps}), flush=True)
        return
    if args.prefill_only:
        print(json.dumps(prefill_steps(pkg, dev)), flush=True)
        return
    if args.draft_only:
        print(json.dumps(draft_steps(pkg, dev)), flush=True)
        return
    if args.only == "config5_attention":
        print(json.dumps(config5_step(pkg, dev, attention_only=True)), flush=True)
        return
    w = build_workload(dev)
    backend = pkg.create_backend("auto", dev, torch.bfloat16, w["d"], w["bs"])
    k = w["k"]
    # Consecutive steps alternate between the pool's two layers (354 MB of KV each), so a
    # step never finds the previous step's KV in the 256 MB MALL.
    kcs = [w["key_pool"][:, layer] for layer in range(2)]
    vcs = [w["value_pool"][:, layer] for layer in range(2)]
    tables, lengths, cu = w["tables"].to(dev), w["lengths"].int().to(dev), w["cu"].to(dev)
    u = w["u"].to(dev)
    ua, uf = u[:, k:2 * k].contiguous(), u[:, 2 * k].contiguous()
    drafts = torch.full((w["n"],), k, dtype=torch.int64, device=dev)
    # draft tokens sampled from q with the draft uniforms (the _draft step)
    w["draft_tokens"] = torch.stack(
        [pkg.categorical(w["qprob"][:, j].contiguous(), u[:, j].contiguous())[0] for j in range(k)], 1)
    dt_tok = w["draft_tokens"]

    rows = w["n"] * w["window"]
    logits = w["target_logits"]
    temp = torch.full((rows,), w["temperature"], device=dev)
    top_k = torch.full((rows,), -1, dtype=torch.int64, device=dev)
    top_p = torch.full((rows,), w["top_p"], device=dev)
    pbuf = {}

    def kv_write(layer=1):
        pkg.store_kv(kcs[layer], vcs[layer], w["k_new"], w["v_new"], w["w_blocks"],
                     w["w_offsets"])

    def attn(layer=1):
        return backend.prefill(w["q"], kcs[layer], vcs[layer], tables, lengths, cu, w["window"])

    def attn_store(layer=1):
        # the two calls above as one launch pair: the attention waves that read a window
        # position store its K/V first
        return backend.prefill_store(w["q"], w["k_new"], w["v_new"], kcs[layer], vcs[layer],
                                     tables, lengths, cu, w["window"])

    all_rows = torch.arange(rows, device=dev)

    def probs():
        # _verify: argmax of every verify row and the distributions of the (all random)
        # rows in one launch, async_speculative.py:678-692
        pbuf["t"], p = pkg.verify_distributions(logits, all_rows, temp, top_k, top_p,
                                                max_top_k=0, apply_top_p=True)
        pbuf["p"] = p.view(w["n"], w["window"], -1)
        return pbuf["p"]

    def accept():
        return pkg.speculative_accept(dt_tok, drafts, w["qprob"], pbuf["p"], ua, uf)

    logits3 = logits.view(w["n"], w["window"], -1)

    def verify():
        # the two calls above in one (targets, distributions and the draft rows'
        # row sums in one launch, then the acceptance); bitwise the same results
        return pkg.verify_accept(logits3, temp, top_k, top_p, dt_tok, drafts, w["qprob"], ua, uf,
                                 max_top_k=0, apply_top_p=True)

    def step(layer=1):
        attn_store(layer)
        verify()

    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    # Graphs of `spg` launches back to back: in-graph kernel boundaries cost ~0,
    # so per-launch timings are not inflated by the per-replay launch overhead.
    spg = max(1, min(args.steps_per_graph, args.steps))
    g_kv, g_attn, g_probs = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    g_acc, g_step, g_ver = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    g_fused = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_kv):
        for i in range(spg):
            kv_write(i % 2)
    with torch.cuda.graph(g_attn):
        for i in range(spg):
            out_attn = attn(i % 2)
    with torch.cuda.graph(g_fused):
        for i in range(spg):
            out_fused = attn_store(i % 2)
    with torch.cuda.graph(g_probs):
        for _ in range(spg):
            out_probs = probs()
    with torch.cuda.graph(g_acc):
        for _ in range(spg):
            out_acc = accept()
    with torch.cuda.graph(g_ver):
        for _ in range(spg):
            out_ver = verify()
    with torch.cuda.graph(g_step):
        for i in range(spg):
            step(i % 2)
    for _ in range(max(1, args.warmup // spg)):
        g_step.replay()
    torch.cuda.synchronize()
    if args.only:
        graph = {"kv_write": g_kv, "attention": g_attn, "attention_store": g_fused,
                 "probs": g_probs,
                 "accept": g_acc, "verify": g_ver}[args.only]
        for _ in range(max(1, args.steps // spg)):
            graph.replay()
        torch.cuda.synchronize()
        print(json.dumps({"only": args.only, "launches": max(1, args.steps // spg) * spg}), flush=True)
        return

    # ---- timed region: exactly K whole verify steps
    replays = -(-args.steps // spg)
    steps = replays * spg
    t0 = time.perf_counter()
    for _ in range(replays):
        g_step.replay()
    torch.cuda.synchronize()
    step_s = (time.perf_counter() - t0) / steps

    # ---- per-launch durations with HIP events on the launch stream, queue pre-filled:
    # the median over `reps` graph replays of spg launches each
    def launch_time(graph, reps=50):
        s = torch.cuda.current_stream()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        torch.cuda._sleep(50_000_000)  # keep the GPU busy while the host enqueues
        for a, b in ev:
            a.record(s)
            graph.replay()
            b.record(s)
        torch.cuda.synchronize()
        times = sorted(a.elapsed_time(b) for a, b in ev)
        return times[len(times) // 2] / 1e3 / spg

    t_kv = launch_time(g_kv)
    t_attn = launch_time(g_attn)
    t_fused = launch_time(g_fused)
    t_probs = launch_time(g_probs)
    t_acc = launch_time(g_acc)
    t_ver = launch_time(g_ver)

    # ---- correctness of the measured outputs against an eager run
    eager_attn = attn((spg - 1) % 2)
    eager_probs = probs()
    eager_acc = accept()
    eager_ver = verify()
    torch.cuda.synchronize()
    assert torch.equal(eager_attn, out_attn)
    # the fused store + attention: the same output (the pool already holds the window's
    # K/V from the warmup, and stores of the same bytes change nothing)
    assert torch.equal(eager_attn, out_fused)
    assert torch.equal(eager_probs, out_probs)
    for a, b in zip(eager_acc, out_acc):
        assert torch.equal(a, b)
    # the fused verify round: bitwise the separate calls' results
    assert torch.equal(out_ver[0], pbuf["t"]) and torch.equal(out_ver[1], eager_probs)
    for a, b in zip(out_ver[2], eager_acc):
        assert torch.equal(a, b)

    # the round's bookkeeping after the acceptance: the random requests' outcome merged
    # into the (here all-random) round, async_speculative.py:735-746
    n_req, win = w["n"], w["window"]
    m_req = torch.arange(n_req, device=dev)
    m_rows = torch.arange(n_req * win, device=dev)
    m_ranks = m_req.repeat_interleave(win)
    m_offs = torch.arange(win, device=dev).repeat(n_req)
    m_zero = torch.zeros(n_req, dtype=torch.int64, device=dev)
    m_starts = lengths.long() - win
    t_merge, _ = _graph_time(lambda: pkg.merge_random_round(
        out_ver[0], m_zero, m_zero, m_starts, dt_tok[:, 0], out_ver[2], m_req, m_rows, m_ranks,
        m_offs))

    a_bytes, p_bytes, c_bytes = attention_bytes(w), probs_bytes(w), accept_bytes(w)
    kv_bytes = kv_write_bytes(w)
    achieved = a_bytes / t_attn / 1e9
    tokens = w["n"] * w["window"]
    traffic, traffic_rec = measured_traffic()
    result = {
        "metric": METRIC,
        "value": round(tokens / step_s, 1),
        "unit": "verified tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random KV, q and logits; no model or dataset)",
        "config": {
            "workload": "config3 verify step: window KV write fused into the attention launch, packed q_len=5 causal window, 16q/4kv heads, D=128, "
                        "bf16 SHARED KV, batch 32, ctx U[1024,8192]; target argmax and distributions from "
                        "fp32 logits (T=0.7, top-p 0.9) and acceptance, V=49152",
            "batch": w["n"], "window": w["window"], "q_heads": w["hq"], "kv_heads": w["hkv"],
            "head_dim": w["d"], "block_size": w["bs"], "vocab": w["vocab"],
            "ctx_sum": int(w["lengths"].sum()),
        },
        "hbm_frac_step": round((kv_bytes + a_bytes + p_bytes + c_bytes) / step_s / 1e9 / PEAK_HBM_GBS, 4),
        "kv_write_ms": round(t_kv * 1e3, 4),
        "attention_ms": round(t_attn * 1e3, 4),
        "attention_with_kv_store_ms": round(t_fused * 1e3, 4),
        "probs_ms": round(t_probs * 1e3, 4),
        "accept_ms": round(t_acc * 1e3, 4),
        "verify_accept_ms": round(t_ver * 1e3, 4),
        "merge_random_round_ms": round(t_merge * 1e3, 4),
        "steps_per_graph": spg,
        "part_times": "median of 50 graph replays of steps_per_graph launches; steps and "
                      "attention launches alternate between two 354 MB KV layers (> the 256 MB MALL)",
        "roofline": {
            "kernel": "attention launch (rlt_attn_mfma_kernel + rlt_merge_kernel)",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4),
            "traffic": traffic,
            "traffic_source": ("profiles/verify_step_config3_hbm_traffic.md (bytes per launch, "
                               f"measured at commit {traffic_rec.get('measured_at_commit')}, kernel "
                               f"sources {traffic_rec.get('kernel_source_digest')}: "
                               + ("this build's)" if traffic is not None else
                                  "not this build's, so not reported)")),
            "algorithmic_bytes": a_bytes,
        },
    }
    if not args.no_secondary:
        # the compensated P V option (the reference's compensate=True packed kernel) on the
        # same launches, next to the plain kernel in the same harness (alternating layers)
        comp = pkg.MI355XPagedAttention(compensate=True)
        flip = {"i": 0}

        def alternating(kernel):
            flip["i"] ^= 1
            return kernel.prefill(w["q"], kcs[flip["i"]], vcs[flip["i"]], tables, lengths, cu,
                                  w["window"])
        t_plain2, _ = _graph_time(lambda: alternating(backend.kernel), reps=21, per_graph=10)
        t_comp, _ = _graph_time(lambda: alternating(comp), reps=21, per_graph=10)
        result["compensated_attention"] = {"us": round(t_comp * 1e6, 1),
                                           "plain_us_same_harness": round(t_plain2 * 1e6, 1)}
    if not args.no_config2:
        del g_kv, g_attn, g_fused, g_probs, g_acc, g_step, g_ver
        result["config2_decode_attention"] = config2_decode(pkg, dev)
    if not args.no_secondary:
        result["batch64_ctx4096_verify"] = target_step(pkg, dev)
        torch.cuda.empty_cache()
        result["config4_verify"] = config4_step(pkg, dev)
        torch.cuda.empty_cache()
        result["config5_verify"] = config5_step(pkg, dev)
        torch.cuda.empty_cache()
        result["prefill"] = prefill_steps(pkg, dev)
        torch.cuda.empty_cache()
        result["draft_step"] = draft_steps(pkg, dev)
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
