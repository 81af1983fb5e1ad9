"""Every name the reference's callers import from the hot-path modules exists here with the
reference's signature.

The table `tests/golden/reference_imports.json` is written by
`tests/golden/make_import_table.py`, which parses (never imports) the reference's `wanx/`,
`zimg/` and `sinkattention/` sources: each row is one `from <module> import <name>` with every
file:line that imports it (e.g. `wanx/runtime/inference.py:23` for the two timing helpers).
`sinkattention.*` rows are served by the alias package, `wanx.runtime.sink_sparse_wan` rows by
`sinkattn_amd.wan_runtime` and `zimg.runtime.sink_sparse_zimage` rows by
`sinkattn_amd.zimage_runtime`.

Also the two timing helpers the Wan inference CLI imports, on hand-built summaries
(sinkattention/timing.py:103-169)."""
import ast
import dataclasses
import importlib
import inspect
import json
from pathlib import Path

import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
TABLE = json.loads((GOLDEN / "reference_imports.json").read_text())
REFERENCE = Path("/root/reference")


def _row_id(row):
    return f"{row['module']}.{row['name']}"


def _value(src, module):
    """A default-value string of the table as a Python value: a literal (ast.literal_eval),
    or else a bare identifier resolved on the serving module.  Nothing else is evaluated:
    the strings come from parsing untrusted source."""
    try:
        return ast.literal_eval(src)
    except (ValueError, SyntaxError):
        pass
    if not src.isidentifier():
        raise AssertionError(f"default value {src!r} is neither a literal nor a name")
    assert hasattr(module, src), f"default value name {src} is not defined on {module.__name__}"
    return getattr(module, src)


def _check_params(obj, exp, module):
    params = list(inspect.signature(obj).parameters.values())
    assert [p.name for p in params] == [e[0] for e in exp]
    assert [p.kind.name for p in params] == [e[1] for e in exp]
    for p, (name, _, default_src) in zip(params, exp):
        if default_src is None:
            assert p.default is inspect.Parameter.empty, name
        else:
            assert p.default == _value(default_src, module), name


@pytest.mark.parametrize("row", TABLE, ids=_row_id)
def test_reference_import_resolves_with_reference_signature(row):
    module = importlib.import_module(row["serving_module"])
    assert hasattr(module, row["name"]), f"{row['name']} imported at {row['imported_at']}"
    obj = getattr(module, row["name"])
    d = row["definition"]
    if d["kind"] == "function":
        assert callable(obj)
        _check_params(obj, d["params"], module)
    elif d["kind"] == "class":
        assert inspect.isclass(obj)
        for meth, params in d["methods"].items():
            _check_params(getattr(obj, meth), params, module)
        if "fields" in d:
            fields = {f.name: f for f in dataclasses.fields(obj)}
            assert list(fields) == [f[0] for f in d["fields"]]
            for name, default_src in d["fields"]:
                f = fields[name]
                if default_src is None:
                    assert f.default is dataclasses.MISSING and f.default_factory is dataclasses.MISSING
                else:
                    assert f.default == _value(default_src, module), name
    elif d["kind"] == "constant":
        assert obj == _value(d["value"], module)
    else:
        pytest.fail(f"unhandled kind {d['kind']}")


def test_every_caller_file_of_the_drop_in_is_in_the_table():
    seen = {site.rsplit(":", 1)[0] for row in TABLE for site in row["imported_at"]}
    for caller in ("wanx/runtime/inference.py", "wanx/runtime/modify_wan.py",
                   "wanx/runtime/sink_sparse_wan.py", "wanx/offline/calibrate_sink_sparse.py",
                   "zimg/runtime/sink_sparse_zimage.py", "zimg/runtime/inference.py",
                   "zimg/offline/calibrate_sink_sparse.py", "sinkattention/__init__.py"):
        assert caller in seen, caller


@pytest.mark.skipif(not REFERENCE.is_dir(), reason="reference sources not present on this machine")
def test_table_is_current_with_the_reference_sources():
    import sys
    sys.path.insert(0, str(GOLDEN))
    try:
        import make_import_table
    finally:
        sys.path.pop(0)
    assert make_import_table.build(REFERENCE) == TABLE


# ---- timing helpers -------------------------------------------------------------------------

def _summary(total, sections, *, enabled=True, label="wan"):
    return {"enabled": enabled, "label": label, "num_records": len(sections),
            "by_section": {k: {"total_ms": v, "mean_ms": v, "count": 1} for k, v in sections.items()},
            "total_ms": total}


def test_extract_attention_time_ms():
    from sinkattention.timing import extract_attention_time_ms as f
    assert f(None) is None
    assert f({}) is None
    assert f(_summary(9.0, {"inner_total": 4.0}, enabled=False)) is None
    assert f(_summary(9.0, {"inner_total": 4.0, "sparse": 3.0})) == 4.0
    # first preferred section that exists wins; a section without total_ms is passed over
    s = _summary(9.0, {"sparse": 3.0, "mix": 1.5})
    s["by_section"]["inner_total"] = {"count": 2}
    assert f(s, preferred_sections=("missing", "inner_total", "mix", "sparse")) == 1.5
    # no preferred section: the summary total, or None when that is absent too
    assert f(_summary(9.0, {"sparse": 3.0})) == 9.0
    s = _summary(None, {"sparse": 3.0})
    assert f(s) is None
    del s["total_ms"]
    assert f(s) is None
    assert isinstance(f(_summary(7, {})), float)


def test_aggregate_timing_summaries():
    from sinkattention.timing import aggregate_timing_summaries as agg
    assert agg([]) is None
    assert agg([None, _summary(1.0, {"a": 1.0}, enabled=False), {}]) is None
    a = _summary(10.0, {"inner_total": 6.0, "mix": 1.0}, label="b")
    b = _summary(20.0, {"inner_total": 12.0, 7: 2.0}, label="a")
    c = _summary(None, {"inner_total": 3.0}, label="")
    c["by_section"]["mix"] = {"count": 1}            # no total_ms: skipped
    r = agg(iter([a, None, b, c]))
    assert r["count"] == 3
    assert r["labels"] == ["a", "b"]
    assert r["mean_total_ms"] == 15.0 and r["max_total_ms"] == 20.0
    assert list(r["mean_by_section_ms"]) == ["7", "inner_total", "mix"]
    assert r["mean_by_section_ms"] == {"7": 2.0, "inner_total": 7.0, "mix": 1.0}
    assert r["max_by_section_ms"] == {"7": 2.0, "inner_total": 12.0, "mix": 1.0}
    assert r["total_by_section_ms"] == {"7": 2.0, "inner_total": 21.0, "mix": 1.0}
    only_none = agg([_summary(None, {})])
    assert only_none["mean_total_ms"] is None and only_none["max_total_ms"] is None
    assert only_none["mean_by_section_ms"] == {}


def test_collector_summary_feeds_the_helpers():
    from sinkattention.timing import (AttentionTimingCollector, aggregate_timing_summaries,
                                      extract_attention_time_ms)
    col = AttentionTimingCollector(label="layer0", enabled=True)
    if not __import__("torch").cuda.is_available():
        for name in ("inner_total", "sparse", "inner_total"):
            with col.section(name):
                pass
        s = col.summarize()
        assert s["by_section"]["inner_total"]["count"] == 2
        assert extract_attention_time_ms(s) == s["by_section"]["inner_total"]["total_ms"]
        agg = aggregate_timing_summaries([s, col.summarize()])
        assert agg["count"] == 2 and agg["labels"] == ["layer0"]
    off = AttentionTimingCollector(label="x", enabled=False).summarize()
    assert extract_attention_time_ms(off) is None and aggregate_timing_summaries([off]) is None
