"""ctypes declarations of the per-wrapper entry points (filled in as they land)."""


def declare(lib) -> None:
    return None
