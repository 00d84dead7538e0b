"""The seeded generator of the reference's known-answer tests (tests/forward-check.mjs:81,133,254):
seed = Math.imul(seed, 1103515245) + 12345 (32 bits), next() = seed >>> 8."""


class Lcg:
    def __init__(self, seed):
        self.seed = seed & 0xFFFFFFFF

    def next(self):
        self.seed = (self.seed * 1103515245 + 12345) & 0xFFFFFFFF
        return self.seed >> 8
