"""Error types of the OpenPacho API (reference: exceptions.py:4-13).

The three classes keep the reference's names and base classes so that code
catching them keeps working after switching to this package.
"""


class BackendUnavailableError(RuntimeError):
    """The requested runtime, library or device cannot be used."""


class UnsupportedDtypeError(TypeError):
    """A dtype is outside the supported set or the device's capabilities."""


class BackendMismatchError(ValueError):
    """An operation mixes arrays owned by different backends or devices."""
