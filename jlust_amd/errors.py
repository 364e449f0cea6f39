"""Exception types of the JLUST API (src/errors.jl:1-9), raised by the host
mirror and mapped from the C ABI's status codes."""


class JLUSTError(Exception):
    """Base class of every error this package raises."""


class InvalidTensorFormat(JLUSTError):
    pass


class InvalidLevelAccess(JLUSTError):
    pass


class UnsupportedFormat(JLUSTError):
    def __init__(self, fmt, backend, detail=""):
        self.format, self.backend = fmt, backend
        msg = f"UnsupportedFormat: {fmt} not supported by {backend}"
        super().__init__(msg + (f" ({detail})" if detail else ""))


class UnsupportedIndexType(JLUSTError):
    def __init__(self, T, backend, detail=""):
        self.T, self.backend = T, backend
        msg = f"UnsupportedIndexType: {T} not supported by {backend}"
        super().__init__(msg + (f" ({detail})" if detail else ""))


class UnsupportedValueType(JLUSTError):
    def __init__(self, T, backend, detail=""):
        self.T, self.backend = T, backend
        msg = f"UnsupportedValueType: {T} not supported by {backend}"
        super().__init__(msg + (f" ({detail})" if detail else ""))


class IndexOriginMismatch(JLUSTError):
    def __init__(self, have, need):
        self.have, self.need = have, need
        super().__init__(f"IndexOriginMismatch: have {have}, need {need}")


class DeviceMismatch(JLUSTError):
    pass


class IncompatibleExtents(JLUSTError):
    pass


class NonCanonicalStorage(JLUSTError):
    pass


class HIPError(JLUSTError):
    """A HIP runtime failure reported by libjlust_hip.so."""


class NoDevice(HIPError):
    """No usable GPU: the library has no CPU fallback."""
