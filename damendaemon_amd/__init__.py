"""MI355X (gfx950) paged-attention hot path with the damendaemon call signatures.

Modules mirror the reference's: ``kernels`` (attention, rope_batch),
``paged_kernels`` (copy_pages), ``pages`` (PagePool), ``kv_quant``,
``prefill`` (groups), ``attention_budget`` and ``cache_indices``, plus
``packing`` (GPU ragged-batch packer) and ``ragged`` (mixed chunked-prefill
and decode attention over one packed batch).
"""
from .pages import PagePool, PageCapacityError  # noqa: F401
