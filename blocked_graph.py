"""FrozenGraph: a captured forward whose frozen region is re-validated before
every replay.

The drop-in for the reference's blocked_graph.py:4-23. It has the same
constructor `FrozenGraph(pilot, forward, example)`, the same `graph` attribute
(the underlying CapturedForward), and the same `outputs`, `replay()`,
`__call__(value)` and `close()`. `pilot.validate()` runs before the capture
and before every replay or call, so a region that drifted since capture raises
the pilot's ValueError instead of replaying stale state.

The validation is installed as the CapturedForward's pre-launch hook
(thin_backend/graph.py), so it also guards a replay made through `graph`
directly.
"""
from thin_backend.graph import CapturedForward


class FrozenGraph:
    def __init__(self, pilot, forward, example):
        pilot.validate()
        self.pilot = pilot
        self.graph = CapturedForward(forward, example)
        self.graph._before_launch = pilot.validate

    @property
    def outputs(self):
        return self.graph.outputs

    def replay(self):
        return self.graph.replay()

    def __call__(self, value):
        return self.graph(value)

    def close(self):
        self.graph.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False
