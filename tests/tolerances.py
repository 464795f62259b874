"""Numeric bars for block outputs: max-abs <= 2e-3 and
max-abs / max|ref| <= 1e-2, against the f32 CPU oracle. Router ids, logits and dequantized
weights are compared bit for bit."""
MAX_ABS = 2e-3
MAX_REL = 1e-2


def assert_close(got, ref, name, max_abs=MAX_ABS, max_rel=MAX_REL):
    from oracle import moe_oracle as O
    m = O.metrics(got.float().cpu(), ref.float().cpu(), name=name)
    print(f"{name}: max_abs={m['max_abs']:.3e} rel={m['max_abs_over_scale']:.3e} "
          f"1-cos={m['one_minus_cos']:.2e}", flush=True)
    assert m["max_abs"] <= max_abs and m["max_abs_over_scale"] <= max_rel, m
    return m
