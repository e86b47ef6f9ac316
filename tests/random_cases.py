"""Size and seed of the seeded random-shape tests.

TV_RANDOM_CASES overrides each random test's case count and TV_RANDOM_SEED
shifts its seed, so the same tests run as a larger sweep, for example
``TV_RANDOM_CASES=1000 TV_RANDOM_SEED=12000 pytest tests -m gpu -k random``.
Unset, every test keeps its fixed default cases.
"""

import os


def case_count(default):
    return int(os.environ.get("TV_RANDOM_CASES", default))


def case_seed(base):
    return base + int(os.environ.get("TV_RANDOM_SEED", 0))
