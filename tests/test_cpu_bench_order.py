"""bench.py's run(): the per-workload comparisons (GPU launches only) come before the headline, the
headline's own workload last among them and its operands reused by the headline, and the CPU
baselines after every GPU measurement, so the headline's W warm-ups and K timed steps follow
seconds of the same GEMM rather than an idle GPU. Checked on the CPU, the GPU steps replaced by
recorders; the timed steps themselves are headline()'s and unchanged by the order."""
import json


def test_run_order(monkeypatch, capsys):
    import torch
    import bench

    calls = []

    class FakeWorkload:
        def __init__(self, name, ref=None):
            calls.append(("operands", name))
            self.name, self.p = name, "problem " + name

    def compare(w, stream):
        calls.append(("compare", w.name))
        return {"ref_tflops": 1.0, "ref_tile": [128, 128, 2, 2], "tflops": 2.0, "ratio": 2.0}

    def headline(name, steps, warmup, ref, w=None):
        calls.append(("headline", name, w is not None))
        return (w if w is not None else FakeWorkload(name)), {"value": 2.0}

    def cpu_baseline(p):
        calls.append(("cpu", p))
        return {"value": 0.1}

    monkeypatch.setattr(bench, "Workload", FakeWorkload)
    monkeypatch.setattr(bench, "compare", compare)
    monkeypatch.setattr(bench, "headline", headline)
    monkeypatch.setattr(bench, "cpu_baseline", cpu_baseline)
    monkeypatch.setattr(bench, "reference_library", lambda: object())
    monkeypatch.setattr(torch.cuda, "current_stream", lambda: None)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)

    head = "c2"
    bench.run([head], 20, 5, True, True, True)
    others = sorted(n for n in bench.CONFIGS if n != head)

    gpu = [c for c in calls if c[0] in ("compare", "headline")]
    # the comparisons, the headline's workload last; the headline on those operands; then its
    # own comparison against the reference (vs_baseline)
    assert gpu == ([("compare", n) for n in others] + [("compare", head), ("headline", head, True),
                                                       ("compare", head)]), gpu
    assert calls[0] == ("operands", head)  # on the device before the comparisons start
    assert calls.count(("operands", head)) == 1
    last_gpu = max(i for i, c in enumerate(calls) if c[0] in ("compare", "headline"))
    cpu = [i for i, c in enumerate(calls) if c[0] == "cpu"]
    assert cpu and min(cpu) > last_gpu, calls
    assert sorted(c[1] for c in calls if c[0] == "cpu") == sorted(
        "problem " + n for n in bench.CONFIGS)  # one CPU baseline each, the headline's reused

    line = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    assert line["vs_baseline"] == 2.0
    assert line["cpu_baseline"] == {"value": 0.1}
    assert list(line["per_config"]) == sorted(bench.CONFIGS)
    assert all(e["cpu_baseline"] == {"value": 0.1} for e in line["per_config"].values())


def test_run_without_comparisons(monkeypatch, capsys):
    """--no-per-config (and --all): the headline builds its own operands, nothing runs before it."""
    import torch
    import bench

    calls = []

    class FakeWorkload:
        def __init__(self, name, ref=None):
            calls.append(("operands", name))
            self.name, self.p = name, "problem " + name

    def headline(name, steps, warmup, ref, w=None):
        calls.append(("headline", name, w is not None))
        return (w if w is not None else FakeWorkload(name)), {"value": 2.0}

    monkeypatch.setattr(bench, "Workload", FakeWorkload)
    monkeypatch.setattr(bench, "headline", headline)
    monkeypatch.setattr(bench, "cpu_baseline", lambda p: calls.append(("cpu", p)) or {})
    monkeypatch.setattr(torch.cuda, "current_stream", lambda: None)
    monkeypatch.setattr(torch.cuda, "empty_cache", lambda: None)

    bench.run(["c2", "c4"], 20, 5, True, False, False)
    assert calls == [("headline", "c2", False), ("operands", "c2"), ("headline", "c4", False),
                     ("operands", "c4"), ("cpu", "problem c2")], calls
    lines = [json.loads(x) for x in capsys.readouterr().out.strip().splitlines()]
    assert len(lines) == 2 and "per_config" not in lines[0]
