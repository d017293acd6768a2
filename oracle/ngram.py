"""Oracle of spec/ngram.py (test infrastructure, see oracle/__init__.py)."""


def lookup(context: list[int], k: int, max_n: int) -> list[int]:
    """spec/ngram.py:32-45"""
    return lookup_match(context, k, max_n)[0]


def lookup_match(context: list[int], k: int, max_n: int) -> tuple[list[int], int, int]:
    """spec/ngram.py:32-45, also returning (match start, n); (-1, 0) when the
    fallback [context[-1]] * k is taken."""
    for n in range(min(max_n, len(context) - 1), 0, -1):
        suffix = context[-n:]
        for start in range(len(context) - n - 1, -1, -1):
            if context[start:start + n] == suffix:
                source = context[start + n:]
                out: list[int] = []
                for i in range(k):
                    out.append(source[i] if i < len(source) else out[i - len(source)])
                return out, start, n
    return [context[-1]] * k, -1, 0
