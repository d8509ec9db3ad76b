"""TDT's greedy search (core/decoder.c:121-147) over any predict and joint:
the driver the decoder tests run the oracle's and the device's steps through."""


def search(T, predict, joint, blank, durs, max_symbols):
    """core/decoder.c:121-147, TDT's greedy search, over predict(label) and
    joint(t) -> (token, duration index)."""
    toks = []
    predict(blank)
    t, last, lasts = 0, None, 0
    while t < T:
        while True:
            at = t
            k, di = joint(t)
            d = durs[di]
            if k == blank and d == 0:
                d = 1
            t += d
            if not (k == blank and t < T):
                break
        if k == blank:
            break
        toks.append((k, at, durs[di]))
        lasts = lasts + 1 if last == at else 1
        last = at
        predict(k)
        if lasts >= max_symbols and last == t:
            t += 1
    return toks
