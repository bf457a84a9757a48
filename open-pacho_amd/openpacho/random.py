"""Resident pseudorandom arrays with explicit backend and counter ownership.

Philox4x32-10 uses one counter block per output element, in C order, so a
stream does not depend on launch geometry or on how calls split it. NumPy's
default_rng is a different algorithm: equal seeds do not give equal samples.

Generator contract (reference random.py:42-135): a 64-bit seed; the backend
is bound once at construction; calls are serialised and each reserves the
counter range [counter, counter + count) before dispatch, so a failed or
uncertain dispatch burns its range instead of reusing it; empty calls consume
nothing; parameter domains are validated before rounding to the output dtype
and again after it.

Layout of this module: a table of distributions (which raw and rounded
parameter checks each one needs), a counter-range object that owns the
reservation rule, and the Generator that resolves a request against both.
"""

import operator
import secrets
from math import prod
from numbers import Real
from threading import Lock

import numpy as np

from ._array import _shape, ndarray
from .backends import get_backend

__all__ = ["Generator", "default_rng"]

_SEED_LIMIT = 1 << 64  # seeds and counters are 64-bit words
_COUNT_LIMIT = (1 << 31) - 1  # largest output a backend indexes
_FLOATS = frozenset((np.dtype(np.float32), np.dtype(np.float64)))


def _tracing(backend):
    return bool(getattr(backend, "_is_tracing", False))


def _refuse_while_tracing(backend=None):
    if _tracing(get_backend() if backend is None else backend):
        raise NotImplementedError("Random generation is not captured; pass generated arrays as arguments")


# ---- parameter checks ---------------------------------------------------------
# Each distribution names one check on the caller's values (so that a tiny
# negative scale cannot round to a valid -0.0, nor inverted bounds to equal
# ones) and one on the values rounded to the output dtype.


def _accept(first, second):
    return None


def _scale_not_negative(_, scale):
    if isinstance(scale, Real) and scale < 0:
        raise ValueError("scale must be nonnegative")


def _bounds_in_order(low, high):
    if isinstance(low, Real) and isinstance(high, Real) and high < low:
        raise ValueError("uniform requires high >= low")


def _width_finite(low, high):
    with np.errstate(over="ignore"):
        width = high - low
    if high < low or not np.isfinite(width):
        raise ValueError("uniform requires high >= low and finite high-low in output dtype")


_DISTRIBUTIONS = {
    # name: (check of the given values, check of the rounded values)
    "random": (_accept, _accept),
    "uniform": (_bounds_in_order, _width_finite),
    "normal": (_scale_not_negative, _scale_not_negative),
    "exponential": (_scale_not_negative, _scale_not_negative),
}


def _in_dtype(value, dtype, role):
    """The parameter as a finite scalar of the output dtype."""
    if not isinstance(value, Real):
        raise TypeError(f"{role} must be a real scalar")
    problem = f"{role} must be finite and representable in {dtype}"
    try:
        with np.errstate(over="ignore", invalid="ignore"):
            rounded = dtype.type(value)
    except OverflowError as exc:
        raise ValueError(problem) from exc
    if np.isfinite(rounded):
        return rounded
    raise ValueError(problem)


class _CounterRange:
    """The unused part [next, 2**64) of one seed's counter space.

    take(count) hands out the next `count` counters and advances at once, so
    a range is never handed out twice, whatever happens to the dispatch that
    uses it.
    """

    __slots__ = ("next",)

    def __init__(self):
        self.next = 0

    def take(self, count):
        if count > _SEED_LIMIT - self.next:
            raise OverflowError("Philox stream exhausted; create a generator with a new seed")
        first = self.next
        self.next = first + count
        return first


class Generator:
    """A Philox4x32-10 stream pinned to one backend, with a 64-bit seed.

    Calls on one generator are serialised to reserve disjoint counters.
    Not for cryptographic use.
    """

    def __init__(self, seed=None, *, backend=None):
        _refuse_while_tracing()
        self._seed = self._checked_seed(secrets.randbits(64) if seed is None else seed)
        self._backend = get_backend(backend)
        if _tracing(self._backend):
            raise NotImplementedError("Random generation is not captured")
        self._range = _CounterRange()
        self._lock = Lock()

    @staticmethod
    def _checked_seed(seed):
        if isinstance(seed, (bool, np.bool_)):
            raise TypeError("seed must be an integer, not bool")
        seed = operator.index(seed)
        if seed < 0 or seed >= _SEED_LIMIT:
            raise ValueError("seed must be in [0, 2**64)")
        return seed

    # The position of the stream (the next unused counter). Tests and tools
    # move it to reach counter-carry cases.
    @property
    def _counter(self):
        return self._range.next

    @_counter.setter
    def _counter(self, value):
        self._range.next = operator.index(value)

    def random(self, size=None, dtype=np.float64):
        """Uniform samples in [0, 1); size=None returns a resident 0-D array."""
        return self._draw("random", size, dtype, 0, 1)

    def uniform(self, low=0.0, high=1.0, size=None, *, dtype=np.float64):
        """Uniform [low, high), or low when equal; bounds rounded to the output dtype."""
        return self._draw("uniform", size, dtype, low, high)

    def normal(self, loc=0.0, scale=1.0, size=None, *, dtype=np.float64):
        """Normal samples (Box-Muller); scalar location and nonnegative scale."""
        return self._draw("normal", size, dtype, loc, scale)

    def exponential(self, scale=1.0, size=None, *, dtype=np.float64):
        """Exponential samples with nonnegative scalar scale (the mean)."""
        return self._draw("exponential", size, dtype, 0, scale)

    def _output(self, size, dtype):
        dtype = np.dtype(dtype)
        if dtype not in _FLOATS:
            raise TypeError("Random generation requires float32 or float64")
        self._backend.validate_dtype(dtype)
        shape = () if size is None else _shape(size)
        if prod(shape) > _COUNT_LIMIT or max(shape, default=0) > np.iinfo(np.intp).max:
            raise ValueError("Random output exceeds indexing limits")
        return shape, dtype

    def _kernel(self, distribution, dtype):
        """The backend's generator entry point, if it offers this distribution."""
        generate = getattr(self._backend, "random_data", None)
        if generate is None:
            raise NotImplementedError("This backend does not implement random generation")
        offered = getattr(self._backend, "random_distributions", None)
        if offered is None or distribution not in offered(dtype):
            raise NotImplementedError(f"{self._backend.name} does not support {distribution} with {dtype}")
        return generate

    def _draw(self, distribution, size, dtype, first, second):
        _refuse_while_tracing()
        shape, dtype = self._output(size, dtype)
        given, rounded = _DISTRIBUTIONS[distribution]
        given(first, second)
        first = _in_dtype(first, dtype, "first parameter")
        second = _in_dtype(second, dtype, "second parameter")
        rounded(first, second)
        generate = self._kernel(distribution, dtype)
        with self._lock:
            start = self._range.take(prod(shape))
            data = generate(shape, dtype, distribution, self._seed, start, first, second)
        return ndarray._wrap(data, shape, dtype, self._backend)


def default_rng(seed=None, *, backend=None):
    """Construct an independent generator; no global random state or GPU import."""
    return Generator(seed, backend=backend)
