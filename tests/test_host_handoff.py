"""The Q8_K hand-off between a fused producer and the projections that read its result is per host
thread: two model-worker threads (the reference runs one per loaded model,
app/models/worker.py:15-46) never claim each other's blocks. Host-only: CPU tensors stand in for
the producer results and workspaces."""

import threading

import torch

from matricxon_amd.fused_ops import _Handoff


def _result(seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(2, 256, generator=g), torch.empty(64, dtype=torch.uint8)


def test_interleaved_threads_claim_only_their_own_offer() -> None:
    h = _Handoff()
    barrier = threading.Barrier(2)
    results: dict[str, tuple] = {}

    def worker(name: str, seed: int, claim_first: bool) -> None:
        out, ws = _result(seed)
        barrier.wait()
        h.offer(out, ws)           # both threads offer before either claims
        barrier.wait()
        if not claim_first:
            barrier.wait()         # the other thread claims in between
        mine = h.claim(out)
        if claim_first:
            barrier.wait()
        results[name] = (mine is ws, out)

    a = threading.Thread(target=worker, args=("a", 1, True))
    b = threading.Thread(target=worker, args=("b", 2, False))
    a.start(), b.start()
    a.join(), b.join()
    assert results["a"][0] and results["b"][0]
    # neither thread's slot answers for the other thread's result
    assert h.claim(results["a"][1]) is None and h.claim(results["b"][1]) is None


def test_many_interleavings_never_mix_offers() -> None:
    h = _Handoff()
    errors: list[str] = []

    def worker(seed: int) -> None:
        pairs = [_result(seed * 1000 + i) for i in range(8)]
        for it in range(2000):
            out, ws = pairs[it % 8]
            h.offer(out, ws)
            got = h.claim(out)
            if got is not ws:
                errors.append(f"thread {seed} iteration {it}")
                return

    threads = [threading.Thread(target=worker, args=(s,)) for s in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:3]


def test_claim_checks_identity_and_version() -> None:
    h = _Handoff()
    out, ws = _result(3)
    assert h.claim(out) is None                    # nothing offered on this thread
    h.offer(out, ws)
    assert h.claim(out) is ws
    assert h.claim(out.view(512)[:256].view(1, 256)) is None  # fewer elements
    assert h.claim(out.clone()) is None            # other storage
    assert h.claim(out.to(torch.float64)) is None  # not float32
    out.add_(1.0)                                  # in-place write moves the version counter
    assert h.claim(out) is None
    h.offer(out, ws)
    assert h.claim(out.view(2, 256)) is ws         # a view of the same result
    h.clear()
    assert h.claim(out) is None
