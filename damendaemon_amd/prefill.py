"""Token-budget grouping of prefill prompts (damendaemon/prefill.py:4-15).

Order is preserved; a group closes when adding the next prompt would take
it past ``token_budget`` (a single prompt larger than the budget still
forms its own group).
"""


def groups(prompts, slots, token_budget):
    batch, assigned, count = [], [], 0
    for prompt, slot in zip(prompts, slots):
        if batch and count + len(prompt) > token_budget:
            yield batch, assigned
            batch, assigned, count = [], [], 0
        batch.append(prompt)
        assigned.append(slot)
        count += len(prompt)
    if batch:
        yield batch, assigned
