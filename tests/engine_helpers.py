"""Test helpers around the serving engine (GPU tests only)."""
from llm_infer_rust_amd.engine import Engine


class RecordingEngine(Engine):
    """Engine that keeps, per sampling call, the request ids and the logits they were drawn
    from (host copies), so a test can check every draw."""

    def __init__(self, *a, keep_rows=None, **k):
        self.records = []
        self.keep_rows = keep_rows
        super().__init__(*a, **k)

    def _sample_and_commit(self, logits, rows):
        n = len(rows) if self.keep_rows is None else min(len(rows), self.keep_rows)
        self.records.append(([r.uid for r in rows[:n]], logits[:n].float().cpu()))
        before = {r.uid: len(r.output) for r in rows}
        super()._sample_and_commit(logits, rows)
        self.records[-1] += ([r.output[before[r.uid]] for r in rows[:n]],)
