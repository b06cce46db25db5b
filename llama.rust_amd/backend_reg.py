"""Host-side mirror of llama.rust's dynamic backend loading, driving
libggml-hip.so the way ggml_backend_load does (crates/ggml/src/backend.rs:1354-1420):
dlopen -> optional ggml_backend_score (0 = not supported) -> ggml_backend_init
-> api_version check -> registry name, devices and proc addresses.

The struct layouts mirror GgmlBackendRegI / GgmlBackendReg / GgmlBackendDeviceI /
GgmlBackendDevice (crates/ggml/src/sysffi.rs:131-171)."""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
MODULE_PATH = os.path.join(HERE, "libggml-hip.so")
GGML_BACKEND_API_VERSION = 2  # backend.rs:44

DEV_TYPE_NAMES = {0: "cpu", 1: "gpu", 2: "igpu", 3: "accel", 4: "meta"}  # foreign_dev_type, backend.rs:1509-1520


class BackendReg(C.Structure):
    pass


class BackendDevice(C.Structure):
    pass


_RegName = C.CFUNCTYPE(C.c_char_p, C.POINTER(BackendReg))
_RegCount = C.CFUNCTYPE(C.c_size_t, C.POINTER(BackendReg))
_RegDev = C.CFUNCTYPE(C.POINTER(BackendDevice), C.POINTER(BackendReg), C.c_size_t)
_RegProc = C.CFUNCTYPE(C.c_void_p, C.POINTER(BackendReg), C.c_char_p)
_DevStr = C.CFUNCTYPE(C.c_char_p, C.POINTER(BackendDevice))
_DevMem = C.CFUNCTYPE(None, C.POINTER(BackendDevice), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t))
_DevType = C.CFUNCTYPE(C.c_int, C.POINTER(BackendDevice))


class BackendRegI(C.Structure):
    _fields_ = [("get_name", _RegName), ("get_device_count", _RegCount), ("get_device", _RegDev),
                ("get_proc_address", _RegProc)]


BackendReg._fields_ = [("api_version", C.c_int), ("iface", BackendRegI), ("context", C.c_void_p)]


class BackendDeviceI(C.Structure):
    _fields_ = [("get_name", _DevStr), ("get_description", _DevStr), ("get_memory", _DevMem),
                ("get_type", _DevType)]


BackendDevice._fields_ = [("iface", BackendDeviceI), ("reg", C.POINTER(BackendReg)), ("context", C.c_void_p)]


class LoadError(RuntimeError):
    """ggml_backend_load returned None; the message is the loader's log line."""


class Device:
    def __init__(self, ptr):
        self._p = ptr

    @property
    def name(self):
        return self._p.contents.iface.get_name(self._p).decode()

    @property
    def description(self):
        return self._p.contents.iface.get_description(self._p).decode()

    @property
    def memory(self):
        free, total = C.c_size_t(0), C.c_size_t(0)
        self._p.contents.iface.get_memory(self._p, C.byref(free), C.byref(total))
        return free.value, total.value

    @property
    def type(self):
        return DEV_TYPE_NAMES.get(self._p.contents.iface.get_type(self._p), "cpu")

    @property
    def ordinal(self):
        """HIP device ordinal to pass to ghip_init"""
        return int(self._p.contents.context or 0)


class Backend:
    """A loaded module: the registry object ggml_backend_init returned."""

    def __init__(self, handle, reg, path):
        self.handle, self._reg, self.path = handle, reg, path

    @property
    def api_version(self):
        return self._reg.contents.api_version

    @property
    def name(self):
        return self._reg.contents.iface.get_name(self._reg).decode()

    def devices(self):
        it = self._reg.contents.iface
        out = []
        for i in range(it.get_device_count(self._reg)):
            d = it.get_device(self._reg, i)
            if d:
                out.append(Device(d))
        return out

    def proc_address(self, name):
        """the ghip.h entry point of that name, as an integer address (0 if unknown)"""
        return self._reg.contents.iface.get_proc_address(self._reg, name.encode()) or 0


def load(path=MODULE_PATH):
    """ggml_backend_load (backend.rs:1354-1420): refuses a module that is
    missing, scores 0, lacks ggml_backend_init, returns NULL, or reports
    another API version."""
    if not os.path.exists(path):
        raise LoadError(f"ggml_backend_load: failed to load {path}: no such file")
    h = C.CDLL(path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    score = getattr(h, "ggml_backend_score", None)
    if score is not None:
        score.restype, score.argtypes = C.c_int, []
        if score() == 0:
            raise LoadError(f"ggml_backend_load: backend {path} is not supported on this system")
    init = getattr(h, "ggml_backend_init", None)
    if init is None:
        raise LoadError(f"ggml_backend_load: failed to find ggml_backend_init in {path}")
    init.restype, init.argtypes = C.POINTER(BackendReg), []
    reg = init()
    if not reg:
        raise LoadError(f"ggml_backend_load: failed to initialize backend from {path}: "
                        "ggml_backend_init returned NULL")
    if reg.contents.api_version != GGML_BACKEND_API_VERSION:
        raise LoadError(f"ggml_backend_load: failed to initialize backend from {path}: incompatible API version "
                        f"(backend: {reg.contents.api_version}, current: {GGML_BACKEND_API_VERSION})")
    return Backend(h, reg, path)


def init_unscored(path=MODULE_PATH):
    """The registry object without the score gate (for inspection on a host
    with no GPU, where load() refuses the module)."""
    h = C.CDLL(path, mode=os.RTLD_NOW | os.RTLD_LOCAL)
    h.ggml_backend_init.restype, h.ggml_backend_init.argtypes = C.POINTER(BackendReg), []
    return Backend(h, h.ggml_backend_init(), path)
