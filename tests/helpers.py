"""Small helpers shared by the test modules."""


def rel_l2(a, b):
    """||a - b|| / ||b|| in float64 on the CPU."""
    a = a.double().cpu()
    b = b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))
