"""Host-side pieces of ``bench.py`` that need no GPU: the parser of the
rocprofv3 counter files behind ``roofline.traffic``, and the refusal of more
than one GPU."""

from __future__ import annotations

import importlib.util
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_counter_csv_groups_dispatches_per_kernel(tmp_path):
    bench = _bench()
    sub = tmp_path / "host" / "123"
    sub.mkdir(parents=True)
    header = "Correlation_Id,Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n"
    rows = [
        '1,1,"void dsv4::expert_decode_kernel<1, 4>(dsv4::DecodeArgs)",FETCH_SIZE,100.5\n',
        '2,2,"void dsv4::expert_decode_kernel<2, 4>(dsv4::DecodeArgs)",FETCH_SIZE,7.0\n',
        '3,3,"void dsv4::expert_decode_kernel<1, 4>(dsv4::DecodeArgs)",FETCH_SIZE,99.5\n',
        '4,4,__amd_rocclr_copyBuffer,FETCH_SIZE,262144.0\n',
    ]
    (sub / "run_counter_collection.csv").write_text(header + "".join(rows))
    (tmp_path / "run_agent_info.csv").write_text("Node_Id\n1\n")
    per = bench.read_counter_csv(tmp_path)
    assert per["void dsv4::expert_decode_kernel<1, 4>(dsv4::DecodeArgs)"] == [100.5, 99.5]
    assert per["void dsv4::expert_decode_kernel<2, 4>(dsv4::DecodeArgs)"] == [7.0]
    assert per["__amd_rocclr_copyBuffer"] == [262144.0]


def test_counter_csv_absent_gives_nothing(tmp_path):
    assert _bench().read_counter_csv(tmp_path) == {}


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_traffic_passes_fall_back_without_the_profiler(monkeypatch):
    """No rocprofv3 on the host: the in-run counter passes return None, and
    the bench then reports the committed figure (`traffic_from_profile`)."""

    import shutil
    import types

    bench = _bench()
    monkeypatch.setattr(shutil, "which", lambda name: None)
    args = types.SimpleNamespace(tokens=64, pool=16, seed=0)
    assert bench.measure_traffic(args, lambda d: 1.0) is None
    fallback = bench.traffic_from_profile()
    assert isinstance(fallback, int) and fallback > 0
