"""FrozenGraph: a captured forward whose frozen region is re-validated before
every replay.

The drop-in for the reference's blocked_graph.py:4-23. It has the same
constructor `FrozenGraph(pilot, forward, example)` and the same `outputs`,
`replay()`, `__call__(value)` and `close()`. `pilot.validate()` runs before
the capture and before every replay or call, so a region that drifted since
capture raises the pilot's ValueError instead of replaying stale state.
Here it is CapturedForward with a pre-launch hook (thin_backend/graph.py).
"""
from thin_backend.graph import CapturedForward


class FrozenGraph(CapturedForward):
    def __init__(self, pilot, forward, example):
        pilot.validate()
        self.pilot = pilot
        super().__init__(forward, example)

    def _before_launch(self):
        self.pilot.validate()
