"""The core's autotune cache, for sessions of this backend.

As the reference core keeps it (core/src/tuning.rs:116-290): a session's
kernel choices are measured once for a key (the backend, the device and its
runtime, this library's build, the model, the precision and its numeric
classes, and the bins of the session's token capacity and max_seq) and
handed back to later sessions of the same key as `turbo_backend_tuning.cached`.
Entries live in memory for the process and, when a directory is named (the
`TURBO_AUTOTUNE_CACHE` variable, or `dir`), one JSON file per key, named by
the backend and the first 16 hex digits of the SHA-256 of the key's JSON,
written beside and renamed over, so a reader sees the old file or the new one
whole (tuning.rs:235-290). Only measured entries with finite timings are
taken from disk.

The model's part of the key is its architecture and dtype (what the choice
depends on), where the reference core hashes the bundle's manifest and
weights files: this host side loads models from memory.
"""
import hashlib
import json
import os
import threading
from dataclasses import asdict, dataclass

from . import seam as S

# The packed-token bins' upper edges, as the backend bins a run's tokens
# (tuning.rs:119-126).
BIN_EDGES = (256, 1024, 4096, 16384)

# Budgets: the time a session may spend measuring (include/turbo/turbo.h:549-552).
BUDGET_WITH_DISK_MS = 750
BUDGET_MEMORY_MS = 150


def tcap_bin(tokens):
    """The highest token bin a session of `tokens` packed tokens at most has."""
    return sum(1 for e in BIN_EDGES if e < tokens)


def max_seq_bin(max_seq):
    """max_seq rounded up to a power of two, 64 at least."""
    v = max(64, int(max_seq))
    return 1 << (v - 1).bit_length()


@dataclass(frozen=True)
class TuneKey:
    backend: str
    device_name: str
    arch: str
    runtime_version: str
    library_build: str
    model: str
    precision: int
    compute_dtype: int
    numerics_allowed: int
    tcap_bin: int
    max_seq_bin: int

    def json(self):
        return json.dumps(asdict(self), sort_keys=True).encode()


def model_fingerprint(desc):
    """The model's part of a key: its family, dtype and shape."""
    fields = (desc.family, desc.dtype, desc.layers, desc.hidden, desc.heads, desc.intermediate, desc.vocab_size,
              desc.max_positions, desc.token_types, getattr(desc, "compute_dtype", 0))
    return hashlib.sha256(repr(fields).encode()).hexdigest()[:32]


_build_hash = {}


def library_build(path):
    """The SHA-256 of the built library, so an entry measured on other
    kernels is never taken."""
    st = os.stat(path)
    k = (path, st.st_mtime_ns, st.st_size)
    if k not in _build_hash:
        h = hashlib.sha256()
        with open(path, "rb") as f:
            for chunk in iter(lambda: f.read(1 << 20), b""):
                h.update(chunk)
        _build_hash[k] = h.hexdigest()[:32]
    return _build_hash[k]


class TuneCache:
    """Measured choices by key: in memory, and in `dir` when one is named."""

    def __init__(self, dir=None):
        self.dir = dir if dir is not None else os.environ.get("TURBO_AUTOTUNE_CACHE") or None
        self._map = {}
        self._lock = threading.Lock()

    def budget_ms(self):
        return BUDGET_WITH_DISK_MS if self.dir else BUDGET_MEMORY_MS

    def file(self, key):
        return os.path.join(self.dir, f"{key.backend}-{hashlib.sha256(key.json()).hexdigest()[:16]}.json")

    def get(self, key):
        with self._lock:
            if key in self._map:
                return self._map[key]
            if not self.dir:
                return None
            try:
                with open(self.file(key)) as f:
                    e = json.load(f)
            except (OSError, ValueError):
                return None
            if (e.get("key") != asdict(key) or e.get("source") != S.TURBO_TUNED_MEASURED
                    or not all(isinstance(v, (int, float)) and v >= 0 and v == v and v != float("inf")
                               for v in e.get("timings", {}).values())):
                return None
            self._map[key] = e
            return e

    def put(self, key, choices, timings):
        e = {"key": asdict(key), "choices": choices, "source": S.TURBO_TUNED_MEASURED, "timings": timings}
        with self._lock:
            self._map[key] = e
            if self.dir:
                os.makedirs(self.dir, exist_ok=True)
                path = self.file(key)
                tmp = f"{path}.{os.getpid()}.tmp"
                try:
                    with open(tmp, "w") as f:
                        json.dump(e, f, indent=1, sort_keys=True)
                    os.replace(tmp, path)
                finally:
                    if os.path.exists(tmp):
                        os.remove(tmp)
        return e


def parse_timings(text):
    """'<bin>/<gemm>/<tile>=<ms>' lines into a dict."""
    out = {}
    for line in text.splitlines():
        if "=" in line:
            name, ms = line.rsplit("=", 1)
            try:
                out[name] = float(ms)
            except ValueError:
                pass
    return out
