"""A spq4k context created with SPQ4K_* tuning overrides in effect (the
library reads them once, in spq4k_init), so tests can reach every launch
shape and code path, not only the ones the planner picks for their sizes."""
import os


def context_with(env):
    import spq4k
    saved = {k: os.environ.get(k) for k in env}
    try:
        for k, v in env.items():
            os.environ[k] = str(v)
        return spq4k.Context(0)
    finally:
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
