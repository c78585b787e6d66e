"""Exceptions of the link executor."""


class LinkRuntimeError(RuntimeError):
    """A link cannot run safely; the counterpart of the reference's
    PICRuntimeError (patched_sglang_files/python/sglang/srt/pic_runtime.py:612).
    Messages follow the reference's wording so callers that match on them keep
    working."""
