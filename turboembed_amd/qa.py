"""Extractive QA's encoder step on the device: start and end logits of
every token of a batch of windows, through the model's span head.

As the core runs a QA window batch (reference core/src/qa/session.rs:172-290):
windows are taken max_batch at a time, padded to the longest with the
tokenizer's fill id (type 0, mask 0), and every live token is a range of
its own, so a range's mean is the token's final state. On a model loaded
with its span head (the table's token_head), the range write applies the
head on the device and each range's row is [start, end]. Logits that are
not finite are an error, as there. Building windows from text (the
tokenizer's question and context split) is the caller's.
"""
import numpy as np

from . import seam as S


def span_logits(session, windows, fill_id=0):
    """[(start [n], end [n])] per window, for windows [(ids, types)]."""
    from . import TurboError
    head = session.model.desc.span_head
    if head is None:
        raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 0, "the model was loaded without a span head")
    if head[0].shape[0] != 2:
        raise TurboError(S.TURBO_E_INVALID_ARGUMENT, 0, "a span head has two outputs, start and end")
    out = []
    for at in range(0, len(windows), session.max_batch):
        chunk = windows[at:at + session.max_batch]
        seq = max(len(w) for w, _ in chunk)
        ids = np.full((len(chunk), seq), fill_id, np.int32)
        types = np.zeros_like(ids)
        mask = np.zeros_like(ids)
        ranges = []
        for r, (wi, wt) in enumerate(chunk):
            n = len(wi)
            ids[r, :n], types[r, :n], mask[r, :n] = wi, wt, 1
            ranges += [(r, i, i + 1) for i in range(n)]
        session.write_ranges(ids, mask, ranges, types, normalize=S.TURBO_NORMALIZE_NONE)
        session.run()
        logits = session.read()
        if logits.shape != (len(ranges), 2):
            raise TurboError(S.TURBO_E_INTERNAL, 0, "QA encoder returned an unexpected state shape")
        if not np.isfinite(logits).all():
            raise TurboError(S.TURBO_E_INTERNAL, 0, "QA head logits overflow F32")
        k = 0
        for wi, _ in chunk:
            n = len(wi)
            out.append((logits[k:k + n, 0].copy(), logits[k:k + n, 1].copy()))
            k += n
    return out
