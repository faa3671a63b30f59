"""Import name of the reference extension (``import flash_attn_wmma``).

Re-exports the two operators of the MI355X build so code written against
thebigblender/FlashLite runs unchanged from the repository root.
"""

from flashlite_amd import forward_flash2, forward_naive  # noqa: F401

__all__ = ["forward_flash2", "forward_naive"]
