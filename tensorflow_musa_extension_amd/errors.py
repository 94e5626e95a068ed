"""Exceptions raised by the ops, named after tf.errors so that callers written
against TensorFlow's op errors read the same (TF_Code values)."""
from . import _lib


class OpError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code
        self.message = message


class InvalidArgumentError(OpError):
    pass


class FailedPreconditionError(OpError):
    pass


class UnimplementedError(OpError):
    pass


class InternalError(OpError):
    pass


class UnknownError(OpError):
    pass


_BY_CODE = {
    _lib.INVALID_ARGUMENT: InvalidArgumentError,
    _lib.FAILED_PRECONDITION: FailedPreconditionError,
    _lib.UNIMPLEMENTED: UnimplementedError,
    _lib.INTERNAL: InternalError,
}


def raise_for_status(status):
    """Raises the tf.errors-style exception for a non-OK TFMA_Status."""
    if status.code == _lib.OK:
        return
    cls = _BY_CODE.get(status.code, UnknownError)
    raise cls(status.code, status.message.decode(errors="replace"))
