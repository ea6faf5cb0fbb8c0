"""GPU power and utilisation sampler: the counterpart of the reference's
aneperf sampler (bench_test.go:62-66, 169-182: Start() before a measured
call, Stop(snapshot) after it, ReportMetrics with ane-watts and
ane-compute-%), for the MI355X the engine runs on.

It reads the amdgpu driver's sysfs files of the HIP device (found by its
PCI bus id): hwmon ``power1_input`` (socket power, microwatts) and
``gpu_busy_percent``, polled from a background thread between Start and
Stop.  Where the files are missing (no GPU, another driver) the sampler is
unavailable and Start / Stop return empty results, as the reference's
benchmarks run without aneperf when NewSampler fails.
"""
from __future__ import annotations

import ctypes
import dataclasses
import glob
import os
import threading
import time
from typing import Optional


@dataclasses.dataclass
class Delta:
    """One Start..Stop window."""
    seconds: float = 0.0
    samples: int = 0
    watts_avg: float = 0.0
    watts_max: float = 0.0
    energy_j: float = 0.0
    busy_pct: float = 0.0

    def metrics(self) -> dict:
        """The reported metrics (aneperf's ane-watts / ane-compute-%)."""
        if not self.samples:
            return {}
        return {"gpu-watts": round(self.watts_avg, 1), "gpu-watts-max": round(self.watts_max, 1),
                "gpu-busy-%": round(self.busy_pct, 1), "gpu-joules": round(self.energy_j, 3)}


def _device_dir(device: int) -> Optional[str]:
    try:
        hip = ctypes.CDLL("libamdhip64.so")
        buf = ctypes.create_string_buffer(64)
        if hip.hipDeviceGetPCIBusId(buf, 64, int(device)) != 0:
            return None
        bdf = buf.value.decode().lower()
    except (OSError, AttributeError):
        return None
    d = os.path.join("/sys/bus/pci/devices", bdf)
    return d if os.path.isdir(d) else None


class Sampler:
    """NewSampler / Start / Stop / Close of aneperf for one HIP device."""

    def __init__(self, device: int = 0, interval_s: float = 0.002):
        self.interval = interval_s
        self._power = self._busy = None
        d = _device_dir(device)
        if d:
            for p in sorted(glob.glob(os.path.join(d, "hwmon", "hwmon*", "power1_input"))):
                self._power = p
                break
            b = os.path.join(d, "gpu_busy_percent")
            self._busy = b if os.path.exists(b) else None
        self._thread = None
        self._stop = threading.Event()
        self._rows = []

    @property
    def available(self) -> bool:
        return self._power is not None

    @staticmethod
    def _read(path):
        try:
            with open(path) as f:
                return float(f.read().strip())
        except (OSError, ValueError):
            return None

    def _loop(self):
        while not self._stop.is_set():
            w = self._read(self._power)
            b = self._read(self._busy) if self._busy else None
            if w is not None:
                self._rows.append((time.perf_counter(), w * 1e-6, b))
            self._stop.wait(self.interval)

    def Start(self) -> float:
        """Begins a window; returns its start time (the snapshot)."""
        self.Stop(None)
        self._rows = []
        t0 = time.perf_counter()
        if self.available:
            self._stop.clear()
            self._thread = threading.Thread(target=self._loop, daemon=True)
            self._thread.start()
        return t0

    def Stop(self, snapshot: Optional[float]) -> Delta:
        """Ends the window opened by Start(); averages over its samples.
        The energy covers the whole window: the trapezoids between samples,
        plus the first sample's power held back to the window's start and the
        last one's held on to its end (the thread's start-up gap and the time
        after the last poll)."""
        t_end = time.perf_counter()
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
            self._thread = None
        if snapshot is None:
            return Delta()
        rows = self._rows
        dt = t_end - snapshot
        rows = [r for r in rows if r[0] <= t_end]
        if not rows:
            return Delta(seconds=dt)
        ws = [r[1] for r in rows]
        energy = sum(0.5 * (rows[i][1] + rows[i - 1][1]) * (rows[i][0] - rows[i - 1][0]) for i in range(1, len(rows)))
        energy += rows[0][1] * max(0.0, rows[0][0] - snapshot) + rows[-1][1] * max(0.0, t_end - rows[-1][0])
        busy = [r[2] for r in rows if r[2] is not None]
        return Delta(seconds=dt, samples=len(rows), watts_avg=sum(ws) / len(ws), watts_max=max(ws), energy_j=energy,
                     busy_pct=(sum(busy) / len(busy)) if busy else 0.0)

    def Close(self):
        self.Stop(None)
