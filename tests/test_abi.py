"""The C ABI without a GPU: the library loads, exports every function include/sm_base2.h declares, and the
host-side error paths (which fail before any device call) report the documented codes."""
from __future__ import annotations

import ctypes
import json
import os
import re

import pytest

from conftest import REPO

HEADER = os.path.join(REPO, "include", "sm_base2.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(sm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared()
    for n in ("sm_create", "sm_destroy", "sm_reset", "sm_prefill", "sm_generate", "sm_read", "sm_record_at",
              "sm_last_error", "sm_stage_attend", "sm_plate_product", "sm_profile"):
        assert n in names


def test_library_exports_every_declared_symbol(sm):
    L = sm.lib()
    missing = [n for n in declared() if not hasattr(L, n)]
    assert missing == []


def test_create_reports_io_errors_before_any_device_call(sm, tmp_path):
    with pytest.raises(sm.SmError) as e:
        sm.Machine(str(tmp_path / "no_such_dir"))
    assert e.value.code == -2 and "manifest.json" in str(e.value)
    (tmp_path / "manifest.json").write_text(json.dumps({"banks": [], "log2_768": 1}))
    with pytest.raises(sm.SmError) as e:
        sm.Machine(str(tmp_path))
    assert e.value.code == -2


def test_stage_switches(sm, tmp_path):
    """each stage is int or float (base2.py:10-11); the bits the binding sends are the header's SM_FLOAT_*"""
    with pytest.raises(ValueError):
        sm.Machine(str(tmp_path), gauge="half")
    import re
    from streaming_machine_amd import machine
    hdr = open(os.path.join(REPO, "include", "sm_base2.h")).read()
    bits = dict(re.findall(r"SM_FLOAT_([A-Z]+) = (\d+)", hdr))
    assert {k.lower(): int(v) for k, v in bits.items()} == machine.FLOAT_STAGES
    names = [f[0] for f in machine.SmConfig._fields_]
    assert names[-5:] == ["inv", "float_stages", "top_read", "att_split", "v64"]
    fields = re.search(r"typedef struct \{(.*?)\} sm_config;", re.sub(r"/\*.*?\*/", "", hdr, flags=re.S), re.S).group(1)
    assert re.findall(r"int32_t (\w+);", fields) == names      # the binding's layout is the header's


def test_last_error_is_a_string(sm):
    L = sm.lib()
    assert isinstance(L.sm_last_error(), bytes)


def test_null_arguments(sm):
    L = sm.lib()
    assert L.sm_create(None, None, None) == -1
    assert L.sm_reset(None) == -1
    assert L.sm_generate(None, 1, None) == -1


def test_graph_steps_bounded_before_any_device_call(sm, tmp_path):
    """captured graphs hold at most 16 decode steps: more is refused with SM_E_ARG before the layout is read"""
    with pytest.raises(sm.SmError) as e:
        sm.Machine(str(tmp_path / "no_such_dir"), graph_steps=17)
    assert e.value.code == -1 and "graph_steps" in str(e.value)
