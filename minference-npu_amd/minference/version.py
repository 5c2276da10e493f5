"""Version of the MI355X sparse prefill attention build (API of MInference 0.1.6)."""

_MAJOR = "0"
_MINOR = "1"
_PATCH = "6"
_SUFFIX = "mi355x"

VERSION = f"{_MAJOR}.{_MINOR}.{_PATCH}+{_SUFFIX}"
