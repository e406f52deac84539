"""Profiler regions: roctxProfilerResume / roctxProfilerPause around measured
loops, so that ``rocprofv3 --selected-regions --marker-trace`` records only
the dispatches between them."""
import ctypes


class ProfilerRegions:
    """roctxProfilerResume / roctxProfilerPause around the measured loops.
    Without a profiler attached both calls do nothing; when the roctx library
    is absent the regions are empty statements."""

    def __init__(self):
        self.lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1"):
            try:
                self.lib = ctypes.CDLL(name)
                break
            except OSError:
                continue
        if self.lib is not None:
            for fn in (self.lib.roctxProfilerResume, self.lib.roctxProfilerPause):
                fn.argtypes = [ctypes.c_uint64]
                fn.restype = ctypes.c_int

    def resume(self):
        if self.lib is not None:
            self.lib.roctxProfilerResume(0)

    def pause(self):
        """Called after the region's work has completed on the GPU."""
        if self.lib is not None:
            self.lib.roctxProfilerPause(0)
