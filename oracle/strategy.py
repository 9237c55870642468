"""Procedural restatement of the reference's ring scheduling strategies.

TEST INFRASTRUCTURE: only tests/ may import this module (it checks the library's
closed-form positions, never replaces them).

Follows rust/src/model/attention/strategy.rs step by step:

* :func:`build_assignment`        strategy.rs:53-110 (Vanilla / Striped / ZigZag)
* :func:`build_domain_positions`  strategy.rs:114-121
* :func:`build_inverse_perm`      strategy.rs:129-143
"""
from __future__ import annotations

VANILLA, STRIPED, ZIGZAG = "vanilla", "striped", "zigzag"


def build_assignment(chunks, strategy):
    """a[p] = domain owning global position p (strategy.rs:53-110)."""
    seq_len = sum(chunks)
    if strategy == VANILLA:
        out = []
        for domain, c in enumerate(chunks):
            out.extend([domain] * c)
        return out
    if strategy == STRIPED:
        # one slot per domain with quota left, in domain order, until all are consumed
        sched = []
        remaining = list(chunks)
        while any(c > 0 for c in remaining):
            for domain in range(len(remaining)):
                if remaining[domain] > 0:
                    sched.append(domain)
                    remaining[domain] -= 1
        return [sched[p % len(sched)] for p in range(seq_len)]
    if strategy == ZIGZAG:
        prefix = [c // 2 + c % 2 for c in chunks]
        suffix = [c // 2 for c in chunks]
        out = []
        for domain, n in enumerate(prefix):
            out.extend([domain] * n)
        for domain in reversed(range(len(chunks))):
            out.extend([domain] * suffix[domain])
        return out
    raise ValueError(strategy)


def build_domain_positions(assignment):
    """Ascending positions of every domain (strategy.rs:114-121)."""
    n = max(assignment) + 1 if assignment else 0
    out = [[] for _ in range(n)]
    for p, d in enumerate(assignment):
        out[d].append(p)
    return out


def build_inverse_perm(assignment):
    """inverse[p] = index of p in the domain-major concatenation (strategy.rs:129-143)."""
    positions = build_domain_positions(assignment)
    inverse = [0] * len(assignment)
    base = 0
    for plist in positions:
        for i, p in enumerate(plist):
            inverse[p] = base + i
        base += len(plist)
    return inverse
