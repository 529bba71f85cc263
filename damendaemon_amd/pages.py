"""Host-side ownership of the bounded pool of KV pages.

Same contract as damendaemon/pages.py:4-56 (the scheduler imports
``PageCapacityError`` from here, scheduler.py:739):
  * pages hold ``page_size`` tokens; ``capacity = tokens // page_size``;
  * the free list starts as ``capacity-1, ..., 1, 0`` and is used as a
    stack, so a fresh pool hands out 0, 1, 2, ... (pages.py:16,46);
  * ``resize_many`` validates every request before it changes anything and
    raises ``PageCapacityError`` when the pool cannot cover the growth;
    shrinking returns a slot's tail pages to the free list, growing pops
    pages for it; ``revision`` advances once per slot that changed in each
    of the two phases (pages.py:38-47).
Pure Python: the device-side page table is built from ``pages`` by the
executor (paged.py:36-44) or by ``page_table()`` below.
"""


class PageCapacityError(Exception):
    pass


def _positive_int(x):
    return type(x) is int and x > 0


class PagePool:
    def __init__(self, tokens, slots, context, page_size=16):
        if not all(map(_positive_int, (tokens, slots, context, page_size))):
            raise ValueError('KV token budget must be a page multiple and fit one page per slot')
        if tokens % page_size or tokens < slots * page_size:
            raise ValueError('KV token budget must be a page multiple and fit one page per slot')
        self.page_size = page_size
        self.context = context
        self.capacity = tokens // page_size
        self.pages = [[] for _ in range(slots)]
        self.free = list(range(self.capacity - 1, -1, -1))
        self.revision = 0
        self.high_water_tokens = 0

    def needed(self, tokens):
        """Pages that hold ``tokens`` tokens (ceil division)."""
        if type(tokens) is not int or tokens < 0 or tokens > self.context:
            raise ValueError('invalid KV reservation length')
        return -(-tokens // self.page_size)

    def resize_many(self, requests, replace=False):
        """Resize several slots as one transaction.

        Without ``replace`` a slot never shrinks (decode growth); with it the
        slot is set to exactly the pages its new length needs.
        """
        slots = [slot for slot, _ in requests]
        if len(set(slots)) != len(slots):
            raise ValueError('duplicate KV slot')
        target = {}
        for slot, tokens in requests:
            if type(slot) is not int or slot < 0 or slot >= len(self.pages):
                raise ValueError('invalid KV slot')
            count = self.needed(tokens)
            target[slot] = count if replace else max(count, len(self.pages[slot]))
        growth = sum(count - len(self.pages[slot]) for slot, count in target.items())
        if growth > len(self.free):
            raise PageCapacityError('KV page pool is full')
        for slot, count in target.items():        # release first ...
            owned = self.pages[slot]
            if count < len(owned):
                self.free += owned[count:]
                del owned[count:]
                self.revision += 1
        for slot, count in target.items():        # ... then allocate
            owned = self.pages[slot]
            if count > len(owned):
                for _ in range(count - len(owned)):
                    owned.append(self.free.pop())
                self.revision += 1
        self.high_water_tokens = max(self.high_water_tokens, self.used_tokens)

    def release(self, slot):
        self.resize_many([(slot, 0)], replace=True)

    @property
    def used_tokens(self):
        return (self.capacity - len(self.free)) * self.page_size

    def page_table(self, width=None, device=None):
        """int32 (slots, width) table, unused entries -1 (paged.py:20-21,36-44)."""
        import torch
        width = width if width is not None else -(-self.context // self.page_size)
        table = torch.full((len(self.pages), width), -1, dtype=torch.int32)
        for slot, owned in enumerate(self.pages):
            if owned:
                table[slot, :len(owned)] = torch.tensor(owned, dtype=torch.int32)
        return table if device is None else table.to(device)
