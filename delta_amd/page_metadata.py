"""Page-index packer (same call as DELTA/Engine/DELTA/page_metadata.py:42-70), on the HIP kernel."""
from .kernels import pack_page_indices  # noqa: F401

__all__ = ["pack_page_indices"]
