"""Bound the split-KV scratch of one decode launch (damendaemon/attention_budget.py:4-10).

A query row needs, per head, ``splits`` fp32 partial vectors plus one fp32
log-sum-exp each, and one output vector.
"""


def query_rows(heads, dim, splits, scratch_bytes, output_bytes=4):
    if type(scratch_bytes) is not int or scratch_bytes <= 0:
        raise ValueError('attention scratch budget must be a positive byte count')
    per_row = heads * (splits * (dim + 1) * 4 + dim * output_bytes)
    if scratch_bytes < per_row:
        raise ValueError('attention scratch budget cannot fit one query row')
    return scratch_bytes // per_row
