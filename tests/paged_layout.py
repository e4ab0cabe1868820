"""The paged K/V cache layout of ``mk_decode_paged`` as plain torch indexing (test infrastructure).

Pages are ``[L, num_pages, 8, page_size, 128]``: the rows of positions ``[i * page_size,
(i + 1) * page_size)`` of every layer and K/V head live in page ``table[i]``. These helpers convert
between that layout and the contiguous ``[L, 8, max_seq, 128]`` cache of the reference operator
(/root/reference/model.py:79-87), so a paged launch can be checked against a contiguous one.
"""
import torch


def to_pages(cache, page_size, table, num_pages, fill=float("nan")):
    """Scatter a contiguous cache into a pool of ``num_pages`` pages; pages the table does not use
    hold ``fill`` (NaN by default, so a read from a wrong page shows in the logits)."""
    L, KV, S, D = cache.shape
    assert S % page_size == 0 and len(table) == S // page_size
    pages = torch.full((L, num_pages, KV, page_size, D), fill, dtype=cache.dtype, device=cache.device)
    for i, page in enumerate(table):
        pages[:, int(page)] = cache[:, :, i * page_size:(i + 1) * page_size]
    return pages


def from_pages(pages, table):
    """Gather the pages back into a contiguous ``[L, 8, len(table) * page_size, 128]`` cache."""
    return torch.cat([pages[:, int(page)] for page in table], dim=2)
