"""Exceptions mirroring the reference's argument exceptions.

The reference throws ArgumentException / ArgumentNullException / ArgumentOutOfRangeException before any
work (RT/Q4KDotKernel.cs:77-97, :957-976; RT/Q4KWeight.cs:46-62). The C ABI returns status codes instead;
this module maps them back.
"""


class OverfitArgumentError(ValueError):
    """ArgumentException."""


class OverfitArgumentNullError(OverfitArgumentError):
    """ArgumentNullException."""


class OverfitArgumentOutOfRangeError(OverfitArgumentError):
    """ArgumentOutOfRangeException."""


class OverfitUnsupportedTypeError(OverfitArgumentError):
    """A weight type the entry point does not accept."""


class OverfitInvalidOperationError(RuntimeError):
    """InvalidOperationException: the object's state forbids the call (a context that still owns weights)."""


class OverfitHipError(RuntimeError):
    """The HIP runtime reported an error."""


def raise_for_status(rc: int, lib) -> None:
    if rc == 0:
        return
    msg = lib.ovfq_last_error().decode(errors="replace")
    if rc == -1:
        raise OverfitArgumentNullError(msg)
    if rc == -2:
        raise OverfitArgumentError(msg)
    if rc == -3:
        raise OverfitArgumentOutOfRangeError(msg)
    if rc == -4:
        raise OverfitUnsupportedTypeError(msg)
    if rc == -5:
        raise OverfitInvalidOperationError(msg)
    raise OverfitHipError(f"status {rc}: {msg}")
