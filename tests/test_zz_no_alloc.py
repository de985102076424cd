"""wy_paged_decode_step_noalloc (the decode step whose split partials and merge
counters live in the library's static device array) against
wy_paged_decode_step with a caller workspace (the op
wy_lib::paged_gqa_attention_decode_fused), through the C ABI: outputs and the
appended pages bit-identical, on two calls in a row, the second with a
smaller batch, and a batch over the capacity rejected before any launch; and
the entry point captured into a graph after an eager first call, every replay
bit-identical to the workspace step."""

import ctypes
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

HQ, HKV, D, P = 8, 2, 256, 16


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def case(dev, lens, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    bf = lambda *s: torch.randn(*s, device=dev, generator=g).to(torch.bfloat16)
    B = len(lens)
    max_pages = -(-max(lens) // P) + 1
    num_pages = B * max_pages
    bt = torch.randperm(num_pages, device=dev, generator=g).view(B, max_pages).to(torch.int32)
    return dict(q=bf(B, HQ, D), kn=bf(B, HKV, D), vn=bf(B, HKV, D), gate=bf(B, HQ, D),
                kc=bf(num_pages, HKV, P, D), vc=bf(num_pages, HKV, P, D), bt=bt,
                pos=torch.tensor([n - 1 for n in lens], dtype=torch.int64, device=dev))


def call_noalloc(pkg, w, kc, vc, out, batch=None):
    lib = pkg._lib.load()
    L = pkg._lib
    B = w["q"].shape[0] if batch is None else batch
    return lib.wy_paged_decode_step_noalloc(
        L.ptr(w["q"]), L.strides(w["q"]), L.ptr(w["kn"]), L.ptr(w["vn"]), L.strides(w["kn"]),
        L.strides(w["vn"]), L.ptr(kc), L.ptr(vc), L.strides(kc), L.strides(vc),
        L.ptr(w["bt"]), w["bt"].stride(0), L.ptr(w["pos"]), L.ptr(w["gate"]),
        L.strides(w["gate"]), L.ptr(out), L.strides(out), B, HQ, HKV, D, w["bt"].shape[1],
        pkg.gqa_attention_decode_paged.min_pages_per_split_fused(B, w["bt"].shape[1]),
        ctypes.c_void_p(torch.cuda.current_stream(out.device).cuda_stream))


def reference(pkg, dev, w):
    kc, vc = w["kc"].clone(), w["vc"].clone()
    B = w["q"].shape[0]
    sc = pkg.allocate_split_scratch(HQ, D, batch=B, device=dev)
    out = torch.ops.wy_lib.paged_gqa_attention_decode_fused(
        w["q"], w["kn"], w["vn"], kc, vc, w["bt"], w["pos"], *sc, sc.counters, w["gate"])
    return out, kc, vc


@pytest.mark.parametrize("first,second", [
    ([300, 2048, 129, 17, 1000, 640, 77, 1500], [40, 900, 5]),
    ([4096] * 64, [2000, 33]),                 # at the capacity (64 x 8 rows), then small
])
def test_noalloc_step_equals_workspace_step(pkg, dev, first, second):
    for i, lens in enumerate((first, second)):
        say(f"noalloc decode step call {i}: B={len(lens)} max L={max(lens)}")
        w = case(dev, lens, seed=50 + i + len(lens))
        ref, kc_ref, vc_ref = reference(pkg, dev, w)
        kc, vc = w["kc"].clone(), w["vc"].clone()
        out = torch.empty_like(ref)
        rc = call_noalloc(pkg, w, kc, vc, out)
        torch.cuda.synchronize()
        assert rc == 0, pkg._lib.load().wy_status_string(rc)
        assert torch.equal(out, ref), f"call {i}: output differs"
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"call {i}: pages differ"


def test_noalloc_rejects_batch_over_capacity(pkg, dev):
    say("noalloc decode step over capacity")
    lib = pkg._lib.load()
    cap = lib.wy_paged_decode_step_noalloc_max_rows()
    assert cap == 512
    w = case(dev, [64, 64], seed=7)
    out = torch.empty(2, HQ, D, dtype=torch.bfloat16, device=dev)
    kc, vc = w["kc"].clone(), w["vc"].clone()
    rc = call_noalloc(pkg, w, kc, vc, out, batch=cap // HQ + 1)
    assert rc == -5, rc
    assert b"capacity" in lib.wy_status_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(kc, w["kc"]), "a rejected call must not launch"


def test_noalloc_step_graph_replays(pkg, dev):
    """After an eager call (which resolves the array and clears its counters),
    the entry point is captured; each replay, with eager work in between,
    equals the workspace step bit for bit."""
    say("noalloc decode step under graph capture")
    lens = [700, 64, 1900, 300]
    w = case(dev, lens, seed=91)
    ref, kc_ref, vc_ref = reference(pkg, dev, w)
    kc, vc = w["kc"].clone(), w["vc"].clone()
    out = torch.empty_like(ref)
    assert call_noalloc(pkg, w, kc, vc, out) == 0
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(g, stream=s):
        rcs.append(call_noalloc(pkg, w, kc, vc, out))
    assert rcs == [0]
    for i in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i}: output differs"
        assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref), f"replay {i}: pages differ"
        # eager work between replays: the workspace step on other buffers
        reference(pkg, dev, case(dev, [100, 33], seed=92 + i))
        torch.cuda.synchronize()
