"""bench.py's headline protocol on the CPU: every layer handle a graph
captures has made an eager call first (so its workspace exists and its
last call can be re-launched by the per-kernel graphs), for the driver's
exact arguments and across a grid of steps, warm-up and layer counts.  The
layers and graphs are stand-ins that record what the protocol does and
refuse what the library would refuse."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


class _State:
    capturing = False


class _Layer:
    def __init__(self, state):
        self.state, self.eager, self.last = state, 0, False

    def forward_into(self, x, logits, out):
        if self.state.capturing and self.eager == 0:
            raise RuntimeError("captured a layer call before any eager call on the handle")
        if not self.state.capturing:
            self.eager += 1
        self.last = True

    def forward_stage(self, stage):
        if not self.last:
            raise RuntimeError("stage launch without a previous call")


class _GraphSet:
    def __init__(self, state):
        self.state, self.units = state, {}

    def add(self, name, capture, units):
        self.state.capturing = True
        try:
            capture()
        finally:
            self.state.capturing = False
        self.units[name] = units

    def run(self, reps):
        return {k: {"best_ms": 1.0, "median_ms": 1.0, "reps": reps} for k in self.units}


class _Seq:
    """Stands in for the timed-input tensors: indexing must stay in range."""

    def __init__(self, n):
        self.n = n

    def __len__(self):
        return self.n

    def __getitem__(self, i):
        if not 0 <= i < self.n:
            raise IndexError(i)
        return i


def _run(steps, warmup, n_layers):
    state = _State()
    layers = [(_Layer(state), None) for _ in range(n_layers)]
    total = warmup + 3 * steps
    xs = _Seq(total - warmup)  # bench passes xs[warmup:]
    kb = bench.moe_kernel_bytes(1, bench.TOPK)
    gs = _GraphSet(state)
    res, per_kernel = bench.moe_protocol(layers, xs, xs, None, steps, 3, None, kb, graphset=gs)
    plan = bench.protocol_plan(steps, n_layers, kb)
    assert set(res) == {"layer_a", "layer_b", "layer_c", "gate_up", "down", "mall_resident"}
    assert per_kernel == {k: len(plan[k]) for k in ("gate_up", "down")}
    for name in ("layer_a", "layer_b", "layer_c", "mall_resident"):
        assert len(plan[name]) == steps and gs.units[name] == steps
    for k in ("gate_up", "down"):
        assert len(plan[k]) * kb[k] >= bench.MIN_STREAM_BYTES and len(plan[k]) >= steps
    captured = {li for v in plan.values() for li in v}
    assert all(layers[li][0].eager >= 1 for li in captured)
    return plan


def test_driver_arguments():
    """python3 bench.py --gpus 1 --steps 20 --warmup 5 (default 72 layers):
    the layer graphs capture layers 0..59, the per-kernel graphs layers past
    the 25 that the eager timing touches."""
    plan = _run(20, 5, 72)
    assert plan["layer_b"] == list(range(20, 40)) and plan["layer_c"] == list(range(40, 60))
    assert max(plan["gate_up"]) > 25


@pytest.mark.parametrize("steps", [1, 2, 5, 13, 14, 20, 50, 200])
@pytest.mark.parametrize("warmup", [0, 5, 20])
@pytest.mark.parametrize("n_layers", [8, 25, 40, 72])
def test_protocol_grid(steps, warmup, n_layers):
    plan = _run(steps, warmup, n_layers)
    # disjoint layer ranges whenever the rotation allows it
    if 3 * steps <= n_layers:
        a, b, c = (set(plan[k]) for k in ("layer_a", "layer_b", "layer_c"))
        assert not (a & b or b & c or a & c)
