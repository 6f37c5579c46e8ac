"""Stage events for measurement.

While a ``StageEvents`` recorder is active, gs3d.rasterize records a HIP
event on the current stream (the stream every gs3d_* launch uses) at each
stage boundary of its forward and backward passes, so stage spans can be
taken inside real training steps: camera + projection + SH ("project"),
depth ordering ("order"), grouped binning from the end of the ordering
("bin", which includes any time the device waits for the host to read the
pair totals), forward blend ("render_fwd"), blend VJP ("render_bwd"),
projection + SH VJP ("project_bwd") and camera VJP ("camera_bwd").
"totals_read" is the part of "bin" until the host has the totals (on the
device: the early emission of group items, or idle time without it).  With
no recorder active a boundary costs one global lookup.
"""

import torch

_active = None

# (span, from mark, to mark)
SPANS = (
    ("project", "start", "projected"),
    ("order", "projected", "ordered"),
    ("totals_read", "ordered", "totals_read"),
    ("bin", "ordered", "binned"),
    ("render_fwd", "binned", "blended"),
    ("render_bwd", "backward", "blend_vjp"),
    ("project_bwd", "blend_vjp", "projection_vjp"),
    ("camera_bwd", "projection_vjp", "camera_vjp"),
)


def mark(name: str) -> None:
    rec = _active
    if rec is not None:
        event = torch.cuda.Event(enable_timing=True)
        event.record()
        rec.marks.append((name, event))


class StageEvents:
    """Records stage-boundary events while active (a context manager)."""

    def __init__(self):
        self.marks = []

    def __enter__(self):
        global _active
        _active = self
        return self

    def __exit__(self, *exc):
        global _active
        _active = None
        return False

    def spans(self) -> dict[str, list[float]]:
        """Milliseconds of every occurrence of each span (after the events
        have completed), in recording order."""
        out = {name: [] for name, _, _ in SPANS}
        last = {}
        for name, event in self.marks:
            for span, a, b in SPANS:
                if name == b and a in last:
                    out[span].append(last[a].elapsed_time(event))
            last[name] = event
        return out
