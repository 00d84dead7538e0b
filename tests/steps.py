"""The oracle's decode steps as generateMany takes them (public/llama2_numpy.py:1565-1640, public/forward.js:1831-1890):
the forward pass of the latest token with logits, the repetition penalty over the distinct tokens of the latest 64 of
the history (the token included), then the greedy choice (temperature 0) or the draw with the step's random number;
a stop token ends the steps after it is taken."""
import numpy as np

import oracle_lib as ol


def oracle_steps(ref, history, pos, count, temperature, topp, penalty, randoms, stops=()):
    """count steps of the oracle model ref from history[-1] at pos (history is extended with every token taken):
    (the tokens, the logits of each step as the engine keeps them: penalized where the penalty applies)"""
    ids, logits = [], []
    for i in range(count):
        ref.run([history[-1]], pos + i, True)
        lg = ref.logits()
        if penalty != 1.0:
            lg = ol.penalize(lg, set(history[-64:]), penalty)
        t = int(np.argmax(lg)) if temperature == 0.0 else ol.sample(lg, temperature, topp, randoms[i])
        assert t >= 0, "a step the engine would decline or refuse"
        ids.append(t)
        logits.append(lg)
        history.append(t)
        if t in stops:
            break
    return ids, logits
