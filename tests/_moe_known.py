"""Known-answer MoE inputs: outputs fixed exactly by the reference's roundings (test data).

The reference evaluates every route as (moe.py:75-91)

    g = round(x gate_e^T),  u = round(x up_e^T),  a = round(round(silu(g)) * u),
    y = round(a down_e^T),  route = round(y * round(w)),

and sums the top-k routes left to right with a rounding after every add.  The cases below
isolate one of those roundings each.  The hidden row is x = e_0, and expert e has a single
nonzero entry per weight: gate[e, 0, 0] = g, up[e, 0, 0] = u, down[e, 0, 0] = c.  So g and u
reach the epilogue as exact single products, a_0 and y_0 carry the case, and every other
output element is zero.  A route of y = Y exactly uses g = 32 (silu(32) rounds to 32 in bf16
and fp32), u = Y / 32 and c = 1.

Each case names the value the reference's order and roundings give (``expected``) and the value
one plausible mistake gives instead (``mistake``): that rounding dropped, or the slots summed
in another order.  The values were found by exhaustive search over bf16 operands, keeping only
operands whose exact silu(g), products and sums lie at least 0.2 % of their magnitude away from
a bf16 rounding midpoint, so that an fp32 evaluation of silu cannot land on the other side.
"""

from __future__ import annotations

import torch

BF16 = torch.bfloat16
D = 8  # hidden size
I = 8  # intermediate size
R = 3 * 2.0**-10  # a weight whose route vanishes against 1 when added to it alone


def _y(value):
    """A slot whose y is exactly ``value`` (bf16): g = 32, u = value / 32, c = 1."""
    return (32.0, value / 32.0, 1.0)


# (name, [(g, u, c, w) per slot], expected output[0], value under the mistake named)
CASES = [
    ("silu rounding", [(-0.3046875, 1.5, 1.0, 1.0)], -0.193359375, -0.1943359375),
    ("silu rounding", [(-1.375, 1.75, 1.0, 1.0)], -0.484375, -0.486328125),
    ("silu*up rounding", [(-0.396484375, 1.5, 1.25, 1.0)], -0.296875, -0.298828125),
    ("silu*up rounding", [(3.203125, -1.75, 1.75, 1.0)], -9.375, -9.4375),
    ("weighted route rounding", [(*_y(0.9296875), 0.75), (*_y(1.1953125), 0.625)], 1.4375, 1.4453125),
    ("weighted route rounding", [(*_y(1.9921875), 0.625), (*_y(2.453125), 0.875)], 3.375, 3.390625),
    ("routing weight rounding", [(*_y(1.0859375), 1.504150390625)], 1.640625, 1.6328125),
    ("slot order", [(*_y(1.0), 1.0), (*_y(1.0), R), (*_y(1.0), R)], 1.0, 1.0 + 2.0**-7),
    ("slot order", [(*_y(1.0), R), (*_y(1.0), R), (*_y(1.0), 1.0)], 1.0 + 2.0**-7, 1.0),
]


def known_answer_problem(dtype=BF16):
    """(hidden, weights, selected, gate, up, down, expected) on the CPU for every case at once.

    Token t is case t.  Each slot of each case has its own expert; expert 0 is all zeros and
    pads the shorter cases to the largest top-k (its route is exactly zero, and adding zero
    leaves a partial sum unchanged).  ``weights`` are float32, as routers produce them: the
    kernels round them to the activation dtype."""
    k = max(len(slots) for _, slots, _, _ in CASES)
    T = len(CASES)
    E = 1 + sum(len(slots) for _, slots, _, _ in CASES)
    gate = torch.zeros(E, I, D)
    up = torch.zeros(E, I, D)
    down = torch.zeros(E, D, I)
    hidden = torch.zeros(T, D)
    hidden[:, 0] = 1.0
    weights = torch.full((T, k), 0.5)
    selected = torch.zeros(T, k, dtype=torch.int64)
    expected = torch.zeros(T, D)
    e = 1
    for t, (_, slots, value, _) in enumerate(CASES):
        for s, (g, u, c, w) in enumerate(slots):
            gate[e, 0, 0], up[e, 0, 0], down[e, 0, 0] = g, u, c
            weights[t, s] = w
            selected[t, s] = e
            e += 1
        expected[t, 0] = value
    cast = [x.to(dtype) for x in (hidden, gate, up, down)]
    return cast[0], weights, selected, cast[1], cast[2], cast[3], expected.to(dtype)


def midpoint_margin(x: torch.Tensor) -> torch.Tensor:
    """Distance of each float64 value from the nearest bf16 rounding midpoint, relative to the
    value (1 where the value is a bf16 number).  bf16 is sign-magnitude, so adding one to the
    raw bits of a value steps its magnitude up, for either sign."""
    b = x.to(BF16)
    bd = b.double()
    step = torch.where(bd.abs() < x.abs(), 1, -1).to(torch.int32)
    other = (b.view(torch.int16).to(torch.int32) + step).to(torch.int16).view(BF16).double()
    margin = (x - (bd + other) / 2).abs() / x.abs()
    return torch.where(bd == x, torch.ones_like(margin), margin)


def silu_sweep_problem(u: float = 1.5, dtype=BF16):
    """One expert, top-1, weight 1: token t computes round(round(silu(g_t)) * u) for every bf16
    g_t in [-8, -2^-4] and [2^-4, 8] (hidden row [g_t, 1, 0, ...], gate row [1, 0, ...], up row
    [0, u, 0, ...], down[0, 0] = 1).  Returns the problem and the g values."""
    pos = torch.arange(0x3D80, 0x4100, dtype=torch.int16).view(BF16).float()  # 2^-4 .. 8 (excl.)
    g = torch.cat([-pos.flip(0), pos])
    T = g.numel()
    hidden = torch.zeros(T, D)
    hidden[:, 0] = g
    hidden[:, 1] = 1.0
    gate = torch.zeros(1, I, D)
    gate[0, 0, 0] = 1.0
    upw = torch.zeros(1, I, D)
    upw[0, 0, 1] = u
    down = torch.zeros(1, D, I)
    down[0, 0, 0] = 1.0
    weights = torch.ones(T, 1)
    selected = torch.zeros(T, 1, dtype=torch.int64)
    cast = [x.to(dtype) for x in (hidden, gate, upw, down)]
    return (cast[0], weights, selected, cast[1], cast[2], cast[3]), g
