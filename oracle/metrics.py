"""Comparison metrics (oracle side), modelled on the reference's
算子研究/tools/metrics.py:11-47 (max_abs, rel_l2, finiteness) plus cosine."""
import torch


def compare(actual, expected):
    a = actual.detach().double().cpu().flatten()
    e = expected.detach().double().cpu().flatten()
    finite = bool(torch.isfinite(a).all())
    diff = (a - e).abs()
    denom = e.norm().item()
    cos = torch.nn.functional.cosine_similarity(a, e, dim=0).item() if a.numel() else 1.0
    return {
        "finite": finite,
        "max_abs": diff.max().item() if a.numel() else 0.0,
        "rel_l2": (a - e).norm().item() / denom if denom > 0 else float((a - e).norm().item()),
        "cosine": cos,
        "bitwise": bool(torch.equal(actual.detach().cpu(), expected.detach().cpu().to(actual.dtype))),
    }


# Every assert_close call of a test session: (what, max_abs, bound, cosine,
# cosine bound).  tests/conftest.py prints it at the end of the session, so a
# run's log shows how much of each tolerance the results use.
RECORD = []


def assert_close(actual, expected, max_abs, min_cos=0.9999, what=""):
    m = compare(actual, expected)
    RECORD.append((what, m["max_abs"], max_abs, m["cosine"], min_cos))
    ok = m["finite"] and m["max_abs"] <= max_abs and m["cosine"] >= min_cos
    assert ok, f"{what}: {m} (bound max_abs<={max_abs}, cosine>={min_cos})"
    return m
