"""The host side's autotune cache (turboembed_amd/tuning.py), without a
device: keys, bins, the file per entry, and what is refused from disk
(reference core/src/tuning.rs:116-290)."""
import json
import math

from turboembed_amd import seam as S
from turboembed_amd import tuning as TU


def key(**kw):
    base = dict(backend="rocm", device_name="AMD Instinct MI355X", arch="gfx950", runtime_version="7.2",
                library_build="abc", model="m", precision=S.TURBO_PRECISION_FASTEST, compute_dtype=S.TURBO_DTYPE_F16,
                numerics_allowed=4, tcap_bin=4, max_seq_bin=512)
    base.update(kw)
    return TU.TuneKey(**base)


def test_bins_follow_the_core():
    # tuning.rs:124-135: the highest bin a capacity reaches; max_seq as a power of two, 64 at least.
    assert [TU.tcap_bin(t) for t in (1, 256, 257, 1024, 1025, 4096, 16384, 16385, 32768)] == [0, 0, 1, 1, 2, 2, 3, 4, 4]
    assert [TU.max_seq_bin(s) for s in (1, 64, 65, 512, 513, 8192)] == [64, 64, 128, 512, 1024, 8192]


def test_an_entry_round_trips_through_its_file(tmp_path):
    c = TU.TuneCache(str(tmp_path))
    k = key()
    assert c.get(k) is None
    c.put(k, "gt16k:qkv=256x192,out=auto,ffn1=auto,ffn2=256x192,attn=mfma;forced=none", {"gt16k/qkv/auto": 0.2})
    files = list(tmp_path.iterdir())
    assert len(files) == 1 and files[0].name.startswith("rocm-") and files[0].name.endswith(".json")
    assert len(files[0].name) == len("rocm-") + 16 + len(".json")
    e = TU.TuneCache(str(tmp_path)).get(k)
    assert e["choices"].startswith("gt16k:qkv=256x192")
    # Another key finds nothing.
    assert TU.TuneCache(str(tmp_path)).get(key(tcap_bin=3)) is None


def test_entries_the_core_would_not_take_are_not_taken(tmp_path):
    k = key()
    c = TU.TuneCache(str(tmp_path))
    c.put(k, "x", {"a": 1.0})
    path = c.file(k)
    for change in ({"source": S.TURBO_TUNED_CACHE}, {"timings": {"a": math.inf}}, {"timings": {"a": -1.0}},
                   {"key": dict(json.load(open(path))["key"], precision=1)}):
        with open(path) as f:
            e = json.load(f)
        e.update(change)
        with open(path, "w") as f:
            f.write(json.dumps(e).replace("Infinity", "1e999"))
        assert TU.TuneCache(str(tmp_path)).get(k) is None, change
    with open(path, "w") as f:
        f.write("{not json")
    assert TU.TuneCache(str(tmp_path)).get(k) is None


def test_budgets_follow_the_core(tmp_path):
    assert TU.TuneCache(str(tmp_path)).budget_ms() == 750
    assert TU.TuneCache(None).budget_ms() in (150, 750)


def test_timings_lines_parse():
    assert TU.parse_timings("le256/qkv/auto=0.0123\ngt16k/ffn2/256x192=0.25\n") == {
        "le256/qkv/auto": 0.0123, "gt16k/ffn2/256x192": 0.25}
