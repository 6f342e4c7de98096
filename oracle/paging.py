"""Page-accounting model of the reference caches.

TEST INFRASTRUCTURE ONLY (the checker).

Two models:
* ``IntendedPaging`` -- the semantics the reference's comments and tests
  describe: a 256-token page is allocated the first time any of its positions
  is appended (PagedKvCache.cs:5-8, :41-60; MlaLatentCache.cs:29-43), and
  BytesUsed grows by one page's bytes per allocation (:56, :40).
* ``reference_growth_null_pages`` -- the reference's Ensure as written, which
  grows the page-pointer array by doubling but fills only up to the pages
  needed at that moment (PagedKvCache.cs:45-57).  Later calls compare against
  the array length, so some slots stay null and a sequential Append throws.
"""
from __future__ import annotations

PAGE_TOKENS = 256  # PagedKvCache.cs:14


class IntendedPaging:
    def __init__(self, layers: int, page_bytes: int):
        self.pages = [0] * layers          # pages held per layer
        self.page_bytes = page_bytes
        self.bytes_used = 0
        self.seq_len = 0

    def append(self, layer: int, pos: int) -> None:
        need = (pos + 1 + PAGE_TOKENS - 1) // PAGE_TOKENS
        if need > self.pages[layer]:
            self.bytes_used += (need - self.pages[layer]) * self.page_bytes
            self.pages[layer] = need
        self.seq_len = max(self.seq_len, pos + 1)

    def reset(self) -> None:           # PagedKvCache.cs:72
        self.seq_len = 0

    def truncate(self, n: int) -> None:  # PagedKvCache.cs:76
        if n < self.seq_len:
            self.seq_len = n


def reference_growth_null_pages(tokens: int):
    """Replays PagedKvCache.Ensure (:41-60) for sequential appends 0..tokens-1.

    Returns (first_failing_pos or None, sorted null slot indices at the end)."""
    slots: list = []          # None = never allocated
    for pos in range(tokens):
        pages = (pos + 1 + PAGE_TOKENS - 1) // PAGE_TOKENS
        if len(slots) < pages:
            new_len = max(pages, len(slots) * 2)
            old = len(slots)
            slots = slots + [None] * (new_len - old)
            for i in range(old, pages):
                slots[i] = "page"
        if slots[pos // PAGE_TOKENS] is None:
            return pos, [i for i, s in enumerate(slots) if s is None]
    return None, [i for i, s in enumerate(slots) if s is None]
