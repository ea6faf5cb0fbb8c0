"""ane.perf.Sampler (the aneperf counterpart) on a fake sysfs tree: power
averaged and integrated over the Start..Stop window, busy percent
averaged; without the driver's files it is unavailable and returns empty
results.  CPU only."""
import os
import time

from ane import perf


def test_sampler_on_fake_sysfs(tmp_path, monkeypatch):
    dev = tmp_path / "0000:f4:00.0"
    (dev / "hwmon" / "hwmon0").mkdir(parents=True)
    (dev / "hwmon" / "hwmon0" / "power1_input").write_text("500000000\n")   # 500 W in microwatts
    (dev / "gpu_busy_percent").write_text("80\n")
    monkeypatch.setattr(perf, "_device_dir", lambda device: str(dev))
    s = perf.Sampler(interval_s=0.001)
    assert s.available
    snap = s.Start()
    time.sleep(0.05)
    d = s.Stop(snap)
    s.Close()
    assert d.samples >= 5
    assert abs(d.watts_avg - 500.0) < 1e-6 and d.watts_max == 500.0 and abs(d.busy_pct - 80.0) < 1e-9
    span = d.seconds
    # constant power: the energy is the power times the whole window, start-up
    # gap and tail after the last sample included
    assert abs(d.energy_j - 500.0 * span) <= 1e-9 * 500.0 * span
    m = d.metrics()
    assert m["gpu-watts"] == 500.0 and m["gpu-busy-%"] == 80.0


def test_sampler_without_driver(monkeypatch):
    monkeypatch.setattr(perf, "_device_dir", lambda device: None)
    s = perf.Sampler()
    assert not s.available
    d = s.Stop(s.Start())
    assert d.samples == 0 and d.metrics() == {}
