"""Token-budget grouping of prefill prompts (damendaemon/prefill.py:4-15).

Order is preserved; a group closes when adding the next prompt would take
it past ``token_budget`` (a single prompt larger than the budget still
forms its own group).
"""


def groups(prompts, slots, token_budget):
    """Yield (prompts, slots) groups in order.  A group is closed just before
    the prompt that would take its token count past ``token_budget``; a
    prompt longer than the budget still makes a group of its own."""
    pairs = list(zip(prompts, slots))
    first, tokens = 0, 0
    for i, (prompt, _) in enumerate(pairs):
        if i > first and tokens + len(prompt) > token_budget:
            yield [p for p, _ in pairs[first:i]], [s for _, s in pairs[first:i]]
            first, tokens = i, 0
        tokens += len(prompt)
    if first < len(pairs):
        yield [p for p, _ in pairs[first:]], [s for _, s in pairs[first:]]
