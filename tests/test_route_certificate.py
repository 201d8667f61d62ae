"""The routing certificate behind the logit-key selection (CPU, float32).

The few-token gate/up kernel and the one-launch decode layer select a
token's served routes on the logits instead of the softmax scores, and
take that selection only when a certificate holds (route_dev.h,
``rt_served_winners``):
- every logit is finite;
- each selected route's logit is at least 2^-16 above the next winner's;
- the next winner's logit is within 60 of the largest one.

The claim is that the softmax as the router forms it keeps that order
strictly: float32 ``exp(z - m)``, the float32 sum, then the correctly
rounded division. This file checks the claim on adversarial logit vectors,
with gaps at the 2^-16 threshold at every magnitude up to 60 below the
maximum, and with numpy's float32 arithmetic in place of the device's. It
also checks the converse that makes the certificate necessary: logits one
ulp apart can produce equal scores, and the router's tie rule (lower index
first) then picks a different route than the logit order.
"""

import numpy as np

GAP = np.float32(2.0 ** -16)


def softmax_f32(z):
    """The router's softmax in float32: exp(z - m), the sum, one division."""
    z = z.astype(np.float32)
    m = np.float32(z.max())
    e = np.exp((z - m).astype(np.float32)).astype(np.float32)
    s = np.float32(e.sum(dtype=np.float32))
    return (e / s).astype(np.float32)


def topk_by(key, k):
    """Larger key first, then the lower index (the selection rule)."""
    order = np.lexsort((np.arange(key.size), -key.astype(np.float64)))
    return order[:k]


def certified(z, sel):
    """The certificate on the logit-order winners sel[0..k] (k + 1 of them)."""
    if not np.all(np.isfinite(z)):
        return False
    m = np.float32(z.max())
    for j in range(len(sel) - 1):
        zj, zn = np.float32(z[sel[j]]), np.float32(z[sel[j + 1]])
        if not (np.float32(zj - zn) >= GAP and zn >= np.float32(m - np.float32(60.0))):
            return False
    return True


def test_certified_logit_order_equals_score_order():
    rng = np.random.default_rng(0)
    E, k = 384, 6
    checked = near = 0
    for trial in range(4000):
        z = rng.standard_normal(E).astype(np.float32) * np.float32(rng.choice([0.5, 3.0, 12.0]))
        # adversarial: k + 1 winners spaced at (or just above) the 2^-16 threshold, anywhere up to 60 below
        base = np.float32(rng.uniform(-59.0, 0.0)) + np.float32(z.max())
        steps = GAP * np.float32(rng.choice([1.0, 1.0000001, 1.5, 4.0]))
        idx = rng.choice(E, k + 1, replace=False)
        top = np.float32(base + steps * np.float32(k))
        for j, e in enumerate(idx):
            z[e] = np.float32(top - steps * np.float32(j))
        if rng.random() < 0.5:  # the winners at the top, or far below other experts' logits
            z[np.setdiff1d(np.arange(E), idx)] -= np.float32(rng.uniform(0.0, 70.0))
        sel = topk_by(z, k + 1)
        if not certified(z, sel):
            continue
        checked += 1
        near += int(np.any(np.diff(-z[sel]) <= 2 * GAP))
        s = softmax_f32(z)
        assert np.array_equal(topk_by(s, k), sel[:k]), f"trial {trial}: softmax order differs"
        # strictly ordered, not merely tie-broken the same way
        assert np.all(np.diff(s[sel[:k + 1]]) < 0), f"trial {trial}: equal scores under the certificate"
    assert checked > 1000 and near > 500, (checked, near)


def test_one_ulp_logits_can_tie_in_score_and_reorder():
    """Without the certificate the logit order is not the router's order."""
    E, k = 384, 6
    z = np.full(E, -12.0, dtype=np.float32)
    for j, e in enumerate((10, 11, 12, 13, 14)):
        z[e] = np.float32(5.0 - j)
    z[100] = np.float32(0.5)
    z[200] = np.nextafter(np.float32(0.5), np.float32(1.0))  # the larger logit on the higher index
    s = softmax_f32(z)
    assert s[100] == s[200]  # equal scores after the float32 rounding
    by_score = topk_by(s, k)
    by_logit = topk_by(z, k)
    assert by_score[5] == 100 and by_logit[5] == 200
    assert not certified(z, topk_by(z, k + 1))
