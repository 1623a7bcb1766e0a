"""Test helper: capture work issued on a torch stream into a raw HIP graph and list
its node types (never instantiated or launched), through the process's own HIP
runtime (the copy torch loaded, which the library shares)."""

import ctypes

# hipGraphNodeType (hip_runtime_api.h)
KERNEL, MEMCPY, MEMSET, HOST, GRAPH, EMPTY = 0, 1, 2, 3, 4, 5
MEM_ALLOC, MEM_FREE = 10, 11
CAPTURE_GLOBAL = 0  # hipStreamCaptureModeGlobal: unsafe calls (hipMalloc) fail during capture

_hip = None


def hip_runtime():
    global _hip
    if _hip is None:
        import torch  # noqa: F401  (its HIP runtime is the process's)

        paths = {l.split()[-1] for l in open("/proc/self/maps") if "libamdhip64" in l}
        assert len(paths) == 1, f"expected one HIP runtime in the process, found {sorted(paths)}"
        lib = ctypes.CDLL(paths.pop())
        vp = ctypes.c_void_p
        lib.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        lib.hipStreamEndCapture.argtypes = [vp, ctypes.POINTER(vp)]
        lib.hipGraphGetNodes.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_size_t)]
        lib.hipGraphNodeGetType.argtypes = [vp, ctypes.POINTER(ctypes.c_int)]
        lib.hipGraphDestroy.argtypes = [vp]
        lib.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
        _hip = lib
    return _hip


def capture_node_types(stream, fn):
    """Captures fn() (which must issue its work on torch stream `stream`) in global
    capture mode and returns the graph's node types; the capture is always ended."""
    hip = hip_runtime()
    raw = ctypes.c_void_p(stream.cuda_stream)
    assert hip.hipStreamBeginCapture(raw, CAPTURE_GLOBAL) == 0
    graph = ctypes.c_void_p()
    try:
        fn()
    finally:
        rc = hip.hipStreamEndCapture(raw, ctypes.byref(graph))
    assert rc == 0, f"hipStreamEndCapture returned {rc}"
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * max(1, n.value))()
    assert hip.hipGraphGetNodes(graph, nodes, ctypes.byref(n)) == 0
    types = []
    for i in range(n.value):
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(nodes[i], ctypes.byref(t)) == 0
        types.append(t.value)
    hip.hipGraphDestroy(graph)
    return types


def free_device_bytes() -> int:
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip_runtime().hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value
