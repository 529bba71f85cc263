"""Bound the split-KV scratch of one decode launch (damendaemon/attention_budget.py:4-10).

A query row needs, per head, ``splits`` fp32 partial vectors plus one fp32
log-sum-exp each, and one output vector.
"""


def query_rows(heads, dim, splits, scratch_bytes, output_bytes=4):
    """How many query rows one launch may take within ``scratch_bytes``."""
    if type(scratch_bytes) is not int or scratch_bytes <= 0:
        raise ValueError('attention scratch budget must be a positive byte count')
    fp32 = 4
    per_head = splits * (dim + 1) * fp32 + dim * output_bytes   # partials + lse, then the output row
    rows = scratch_bytes // (heads * per_head)
    if rows == 0:
        raise ValueError('attention scratch budget cannot fit one query row')
    return rows
