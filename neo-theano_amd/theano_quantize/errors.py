"""Exceptions mirroring the reference's error types.

``TheanoError`` variants (crates/theano-types/src/error.rs:7-56) and the
``RocmError`` variants that convert into them
(crates/theano-rocm/src/error.rs:3-73).  libtq.so status codes map as
TQ_EINVAL -> InvalidArgument, TQ_EHIP -> KernelError, TQ_ENOMEM -> OutOfMemory.
"""


class TheanoError(Exception):
    """Base error (TheanoError)."""


class InvalidArgument(TheanoError, ValueError):
    """TheanoError::InvalidArgument / ShapeMismatch."""


class KernelError(TheanoError, RuntimeError):
    """RocmError::KernelError / DriverError (surfaced as TheanoError::RuntimeError)."""


class OutOfMemory(TheanoError, MemoryError):
    """RocmError::OutOfMemory -> TheanoError::OutOfMemory."""


TQ_OK, TQ_EINVAL, TQ_EHIP, TQ_ENOMEM = 0, 1, 2, 3


def raise_for_status(status: int, message: str) -> None:
    if status == TQ_OK:
        return
    if status == TQ_EINVAL:
        raise InvalidArgument(message)
    if status == TQ_ENOMEM:
        raise OutOfMemory(message)
    raise KernelError(message)
