"""Loader for the compiled extension.

Same contract as the reference's ``load_extension`` (tinyinfer/utils/
extension.py:4-14): cached, returns the ``_C`` module, and raises
``RuntimeError`` with a build hint when the module has not been built.
"""

from functools import lru_cache


@lru_cache(maxsize=1)
def load_extension():
    import torch  # noqa: F401  (loads libc10_hip / libtorch that _C links against)
    try:
        from tinyinfer_amd import _C
    except ImportError as exc:
        raise RuntimeError(
            "tinyinfer_amd._C is not built; run: python setup.py build_ext --inplace "
            "(or python -m tinyinfer_amd.build)"
        ) from exc
    return _C
