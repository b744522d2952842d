"""bench.py's command line (host logic, no GPU): which runs also time the
other workloads in child processes (other_configs), and that those children's
flags are valid workloads of their own that start no further children."""
import bench


def test_default_run_times_the_other_workloads(monkeypatch):
    monkeypatch.delenv("ROCPROF_OUTPUT_PATH", raising=False)
    ap = bench.build_parser()
    assert bench.default_workload(ap.parse_args([]))
    assert bench.default_workload(ap.parse_args(["--gpus", "1", "--steps", "5", "--warmup", "2", "--seed", "1"]))
    for flags in (["--config", "c2"], ["--config", "c4"], ["--kv", "e4m3"], ["--q-heads", "24"], ["--no-others"],
                  ["--refabi"], ["--unfused"], ["--with-prep"], ["--verify-kernel"], ["--batch", "32"],
                  ["--pages", "262144"], ["--wg-per-cu", "2"], ["--min-range", "64"]):
        assert not bench.default_workload(ap.parse_args(flags)), flags


def test_no_child_runs_under_the_profiler(monkeypatch):
    monkeypatch.setenv("ROCPROF_OUTPUT_PATH", "/tmp/prof")
    assert not bench.default_workload(bench.build_parser().parse_args([]))


def test_other_configs_are_workloads_without_children(monkeypatch):
    monkeypatch.delenv("ROCPROF_OUTPUT_PATH", raising=False)
    ap = bench.build_parser()
    names = [name for name, _ in bench.OTHER_CONFIGS]
    assert len(set(names)) == len(names)
    for name, flags in bench.OTHER_CONFIGS:
        args = ap.parse_args(["--no-cpu", "--no-traffic", "--no-others"] + flags)
        assert not bench.default_workload(args), name
        # without --no-others too: each is a workload other than the default
        assert not bench.default_workload(ap.parse_args(flags)), name
