"""Dense target distributions on the GPU vs the CPU oracle.

* ``softmax_temp`` (SoftmaxTemp.execute): bf16 rows at the full 151,936
  vocabulary (16-byte vector path); fp32 rows of an odd vocabulary (element
  path); fp16 rows with a row stride wider than the vocabulary; rows with
  masked (-inf) entries.  Probabilities within 1e-5 relative (entries above
  1e-30; smaller ones within 1e-35 absolute) of the reference formula's
  exact value: x = logit / T rounded to fp32 as the reference computes it,
  the softmax of x accumulated in fp64.  (The fp32 oracle's own row sums
  over 151,936 terms round by up to ~1e-5, so it is checked against the same
  values at 1e-4.)
* ``target_probs`` / ``build_dflash_verify_target_probs``: top-k 50 + top-p
  0.95 at the full vocabulary (wavefront scan), top-p only (nucleus larger
  than a record holds: dense support), pure temperature, heavy ties with
  top-k 5 and 1000, min-p, and the reference signature with a sampling-info
  object, including max_top_k below some requests' top-k.  Compared with
  the reference formula evaluated in fp64 (after the fp32 quotient): the
  support (which entries are non-zero) is exact except entries on the top-p
  boundary (exact exclusive prefix mass within 1e-6 of top_p); probabilities
  within 1e-5 relative.
"""

from types import SimpleNamespace

import pytest
import torch

from oracle import verify as ov
from longspark_amd import dense, workloads

pytestmark = pytest.mark.gpu


def assert_probs_close(got, ref, label):
    got = got.cpu().float()
    ref = ref.float()
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert torch.isfinite(got).all(), f"{label}: non-finite output"
    big = ref > 1e-30
    relall = (got - ref).abs() / ref.clamp_min(1e-30)
    rel = relall[big]
    worst = float(rel.max()) if rel.numel() else 0.0
    if worst > 1e-5:
        flat = torch.where(big, relall, torch.zeros_like(relall)).reshape(-1)
        top = torch.topk(flat, 5).indices
        rows = got.shape[-1]
        info = [(int(i) // rows, int(i) % rows, float(ref.reshape(-1)[i]), float(got.reshape(-1)[i]),
                 float(flat[i])) for i in top]
        print(f"{label}: worst entries (row, col, ref, got, rel): {info}")
    assert worst <= 1e-5, f"{label}: max relative error {worst:.3g}"
    assert float((got - ref).abs()[~big].max()) <= 1e-35 if (~big).any() else True, f"{label}: tiny entries differ"


def softmax_exact(logits, temps, rows_per_request):
    """The reference formula (softmax_temp.py:69-84) with the softmax in fp64."""
    t = torch.repeat_interleave(temps.reshape(-1).float(), rows_per_request)
    x = logits.float() / t[:, None]
    return torch.softmax(x.double(), dim=-1).float()


def check_softmax(got, logits, temps, rpr, label):
    exact = softmax_exact(logits, temps, rpr)
    assert_probs_close(got, exact, label)
    oracle = ov.softmax_temp(logits, temps, rpr)
    big = exact > 1e-30
    assert float(((oracle - exact).abs() / exact.clamp_min(1e-30))[big].max()) <= 1e-4


def test_softmax_temp_bf16_full_vocab(dev):
    logits, _ = workloads.greedy_inputs(4, 16, seed=51)
    temps = torch.tensor([0.7, 1.0, 1.3, 0.45])
    print("softmax_temp bf16 4x16 x 151936", flush=True)
    got = dense.SoftmaxTemp.execute(logits=logits.to(dev), temperatures=temps.to(dev), rows_per_request=16)
    torch.cuda.synchronize()
    check_softmax(got, logits, temps, 16, "bf16")


def test_softmax_temp_fp32_odd_vocab_and_masked(dev):
    g = torch.Generator().manual_seed(52)
    logits = 4.0 * torch.randn(6, 30001, generator=g)
    logits[1, ::7] = float("-inf")            # masked entries
    logits[2, :29990] = float("-inf")         # nearly all masked
    temps = torch.tensor([0.8, 1.7, 0.3])
    print("softmax_temp fp32 6 x 30001", flush=True)
    got = dense.softmax_temp(logits=logits.to(dev), temperatures=temps.to(dev), rows_per_request=2)
    torch.cuda.synchronize()
    masked = torch.isneginf(logits)
    assert bool((got.cpu()[masked] == 0).all()), "masked entries must be exactly 0"
    check_softmax(got, logits, temps, 2, "fp32 odd vocab")


def test_softmax_temp_fp16_strided(dev):
    g = torch.Generator().manual_seed(53)
    wide = (3.0 * torch.randn(8, 50000 + 24, generator=g)).to(torch.float16)
    logits = wide[:, 8:8 + 50000]             # row stride wider than the vocabulary, offset start
    temps = torch.tensor([1.1, 0.6])
    print("softmax_temp fp16 strided 8 x 50000", flush=True)
    got = dense.softmax_temp(logits=logits.to(dev), temperatures=temps.to(dev), rows_per_request=4)
    torch.cuda.synchronize()
    check_softmax(got, logits, temps, 4, "fp16 strided")


def test_softmax_temp_bf16_resident_tail_and_masked(dev):
    """A 16-bit row held in registers with 3 trailing entries past its last
    4-entry unit, masked entries, a row that is masked but for its last 4
    entries, and a row stride wider than the vocabulary (16-byte aligned)."""
    g = torch.Generator().manual_seed(54)
    wide = (3.0 * torch.randn(6, 30008, generator=g)).to(torch.bfloat16)
    logits = wide[:, :30003].clone()
    logits[1, ::5] = float("-inf")
    logits[3, :29999] = float("-inf")
    temps = torch.tensor([0.9, 1.4, 0.5])
    print("softmax_temp bf16 6 x 30003 (row stride 30008)", flush=True)
    wide_d = wide.to(dev)
    wide_d[:, :30003] = logits.to(dev)
    got = dense.softmax_temp(logits=wide_d[:, :30003], temperatures=temps.to(dev), rows_per_request=2)
    torch.cuda.synchronize()
    masked = torch.isneginf(logits.float())
    assert bool((got.cpu()[masked] == 0).all()), "masked entries must be exactly 0"
    check_softmax(got, logits, temps, 2, "bf16 resident tail")


def run_target_probs(dev, logits, params, rows_per_request, max_top_k=None, min_p=False):
    got = dense.target_probs(logits=logits.to(dev), temperatures=params.temperatures.to(dev),
                             rows_per_request=rows_per_request, top_ks=params.top_ks.to(dev),
                             top_ps=params.top_ps.to(dev), min_ps=params.min_ps.to(dev) if min_p else None,
                             max_top_k=max_top_k, check=True)
    torch.cuda.synchronize()
    mps = params.min_ps if min_p else torch.zeros_like(params.min_ps)
    ref = ov.target_probs(logits, temperatures=params.temperatures, top_ks=params.top_ks, top_ps=params.top_ps,
                          min_ps=mps, rows_per_request=rows_per_request, compute_dtype=torch.float64)
    return got.cpu(), ref


def check_support(got, ref, logits, params, rows_per_request, label):
    """The non-zero pattern matches the exact reference, except entries on the
    top-p boundary: their exact exclusive prefix mass lies within 1e-6 of
    top_p (a CDF-boundary tie under the tolerance contract)."""
    diff = (got != 0) != (ref != 0)
    for r in diff.any(-1).nonzero().flatten().tolist():
        b = r // rows_per_request
        t, k, tp = float(params.temperatures[b]), int(params.top_ks[b]), float(params.top_ps[b])
        x = (logits[r].float() / t).double()
        order = torch.sort(x, descending=True, stable=True).indices
        keep = order[:min(k, x.numel())]
        p = torch.softmax(x[keep], -1)
        excl = torch.cumsum(p, 0) - p
        where = {int(c): i for i, c in enumerate(keep.tolist())}
        for c in diff[r].nonzero().flatten().tolist():
            assert c in where and abs(float(excl[where[c]]) - tp) <= 1e-6, (
                f"{label}: row {r} entry {c} differs off the top-p boundary "
                f"(exclusive prefix {float(excl[where[c]]) if c in where else None!r}, "
                f"support {int((got[r] != 0).sum())} vs {int((ref[r] != 0).sum())})")


@pytest.mark.parametrize("label,vocab,temp,top_k,top_p,min_p,max_top_k", [
    ("k50 p0.95", workloads.VOCAB, 0.7, 50, 0.95, 0.0, 50),
    ("k50 p0.95 no bound", workloads.VOCAB, 0.7, 50, 0.95, 0.0, None),
    ("top-p 0.9 only", workloads.VOCAB, 1.0, workloads.VOCAB, 0.9, 0.0, None),
    ("pure temperature", 20000, 1.3, 20000, 1.0, 0.0, None),
    ("k40 p0.9 min-p 0.05", workloads.VOCAB, 0.8, 40, 0.9, 0.05, 40),
])
def test_target_probs(dev, label, vocab, temp, top_k, top_p, min_p, max_top_k):
    logits, _ = workloads.greedy_inputs(3, 8, vocab, seed=61)
    params = workloads.SamplingParams.uniform(3, temperature=temp, top_k=top_k, top_p=top_p, min_p=min_p)
    print(f"target_probs {label}", flush=True)
    got, ref = run_target_probs(dev, logits, params, 8, max_top_k=max_top_k, min_p=min_p > 0)
    check_support(got, ref, logits, params, 8, label)
    both = (got != 0) & (ref != 0)
    assert_probs_close(torch.where(both, got, ref), ref, label)


@pytest.mark.parametrize("top_k", [5, 1000])
def test_target_probs_ties(dev, top_k):
    g = torch.Generator().manual_seed(62 + top_k)
    logits = torch.randint(-4, 5, (4 * 4, 2000), generator=g).to(torch.bfloat16)
    params = workloads.SamplingParams.uniform(4, temperature=1.0, top_k=top_k, top_p=0.8)
    print(f"target_probs ties k={top_k}", flush=True)
    got, ref = run_target_probs(dev, logits, params, 4)
    check_support(got, ref, logits, params, 4, f"ties k={top_k}")
    both = (got != 0) & (ref != 0)
    assert_probs_close(torch.where(both, got, ref), ref, f"ties k={top_k}")


def test_build_dflash_verify_target_probs_signature(dev):
    logits, _ = workloads.greedy_inputs(4, 8, seed=63)
    info = SimpleNamespace(temperatures=torch.tensor([[0.7], [1.0], [0.9], [1.2]], device=dev),
                           top_ks=torch.tensor([50, 20, 64, 8], dtype=torch.int32, device=dev),
                           top_ps=torch.tensor([0.95, 1.0, 0.9, 0.8], device=dev),
                           need_top_k_sampling=True, need_top_p_sampling=True)
    print("build_dflash_verify_target_probs", flush=True)
    for max_top_k in (None, 32):
        got = dense.build_dflash_verify_target_probs(next_token_logits=logits.to(dev), sampling_info=info,
                                                     draft_token_num=8, bs=4, max_top_k=max_top_k)
        torch.cuda.synchronize()
        assert got.shape == (4, 8, logits.shape[1])
        ks = info.top_ks.cpu().long()
        if max_top_k is not None:
            ks = ks.clamp(max=max_top_k)
        temps = info.temperatures.cpu().reshape(-1)
        ref = ov.target_probs(logits, temperatures=temps, top_ks=ks, top_ps=info.top_ps.cpu(),
                              min_ps=torch.zeros(4), rows_per_request=8, compute_dtype=torch.float64)
        got = got.reshape(32, -1).cpu()
        params = workloads.SamplingParams(temps, ks.to(torch.int32), info.top_ps.cpu(), torch.zeros(4))
        check_support(got, ref, logits, params, 8, f"max_top_k={max_top_k}")
        both = (got != 0) & (ref != 0)
        assert_probs_close(torch.where(both, got, ref), ref, f"max_top_k={max_top_k}")
