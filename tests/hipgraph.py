"""The few HIP runtime calls the GPU tests need to capture and replay a HIP graph on the library's stream (ctypes over
libamdhip64). Test infrastructure only; the library itself never captures anything."""
import ctypes as C


class Graphs:
    def __init__(self):
        self.L = C.CDLL("libamdhip64.so")
        for n in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
                  "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy"):
            getattr(self.L, n).restype = C.c_int

    def ck(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    def capture(self, stream, fn, instantiate=True):
        """Capture what fn() enqueues on `stream`; returns (fn's result, graph, exec or None)."""
        g, ex = C.c_void_p(), C.c_void_p()
        self.ck(self.L.hipStreamBeginCapture(C.c_void_p(stream), 0), "hipStreamBeginCapture")
        try:
            res = fn()
        finally:
            self.ck(self.L.hipStreamEndCapture(C.c_void_p(stream), C.byref(g)), "hipStreamEndCapture")
        if not instantiate:
            return res, g, None
        self.ck(self.L.hipGraphInstantiate(C.byref(ex), g, None, None, C.c_size_t(0)), "hipGraphInstantiate")
        return res, g, ex

    def replay(self, ex, stream):
        self.ck(self.L.hipGraphLaunch(ex, C.c_void_p(stream)), "hipGraphLaunch")
        self.ck(self.L.hipStreamSynchronize(C.c_void_p(stream)), "hipStreamSynchronize")

    def destroy(self, g, ex):
        if ex is not None:
            self.L.hipGraphExecDestroy(ex)
        self.L.hipGraphDestroy(g)
