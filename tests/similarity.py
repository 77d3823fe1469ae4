"""Comparison gates used by the parity tests.

attention_gate mirrors the reference's attention acceptance policy
(test/Board/PyTorch/wafer_pytorch_board_cases.py:31-33 and
test/Board/PyTorch/wafer_pytorch_board_common.py:59-71, 295-306): cosine
similarity >= 0.9999 and relative L2 <= 0.01 decide acceptance; the
elementwise rtol 0.006 / atol 0.008 check is enforced here as well, which is
stricter than the reference.
"""
import numpy as np

ATT_RTOL, ATT_ATOL, ATT_MIN_COS, ATT_MAX_RELL2 = 0.006, 0.008, 0.9999, 0.01


def stats(actual, expected):
    a = np.asarray(actual, dtype=np.float64).ravel()
    e = np.asarray(expected, dtype=np.float64).ravel()
    na, ne = np.linalg.norm(a), np.linalg.norm(e)
    cos = 1.0 if na == 0 and ne == 0 else float(a @ e / max(na * ne, 1e-300))
    rel = 0.0 if ne == 0 and na == 0 else float(np.linalg.norm(a - e) / max(ne, 1e-300))
    return cos, rel, float(np.max(np.abs(a - e))) if a.size else 0.0


def attention_gate(actual, expected, rtol=ATT_RTOL, atol=ATT_ATOL, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    cos, rel, mx = stats(a, e)
    bad = np.abs(a - e) > atol + rtol * np.abs(e)
    assert cos >= ATT_MIN_COS and rel <= ATT_MAX_RELL2, f"{what}: cosine={cos} relL2={rel} maxabs={mx}"
    assert not bad.any(), f"{what}: {int(bad.sum())}/{a.size} elements outside rtol={rtol} atol={atol}; maxabs={mx}"
    return cos, rel, mx
