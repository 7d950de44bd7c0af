"""Host logic of the fused q/k/v + rope step (llaccel_amd.fusion._GroupRopeStep), no GPU: when the
one-launch entry refuses a call, the two-launch path runs; the fused entry is switched off only when
those two launches take the operands (a refusal that is a property of the graph), and an error of the
call itself propagates and leaves the fused entry on."""
from __future__ import annotations

import pytest

from llaccel_amd import _lib, fusion


class _Rec:
    def __init__(self, log, name, fail=False):
        self.log, self.name, self.fail = log, name, fail

    def __call__(self, M, pos, pd=None):
        self.log.append(self.name)
        if self.fail:
            raise ValueError(f"{self.name}: refused")


class _Group(_Rec):
    lins = [{"in": "x", "K": 896}]
    probs = None

    def fill(self):
        pass


class _Rope(_Rec):
    desc = (object(), object())
    parts = ()

    def _fill(self, *a):
        pass


class _Model:
    _ws = None

    def _buf(self, name):
        return None

    def _stream_handle(self):
        return None


def _step(log, monkeypatch, fused_ok, fallback_fails=False):
    def call(name, *args):
        log.append(name)
        if name == "llhip_linear_group_rope" and not fused_ok:
            raise ValueError("linear_group_rope: refused")

    monkeypatch.setattr(_lib, "call", call)
    monkeypatch.setattr(fusion, "_vp", lambda t: None)
    monkeypatch.setattr(fusion.ctypes, "byref", lambda x: x)
    return fusion._GroupRopeStep(_Model(), _Group(log, "group", fallback_fails), _Rope(log, "rope"))


def test_fused_entry_taken(monkeypatch):
    log = []
    st = _step(log, monkeypatch, fused_ok=True)
    st(512, 0)
    st(512, 0)
    assert log == ["llhip_linear_group_rope"] * 2 and st.fused and st.launched == 2


def test_refusal_of_the_graph_switches_the_fused_entry_off(monkeypatch):
    log = []
    st = _step(log, monkeypatch, fused_ok=False)
    st(512, 0)
    assert log == ["llhip_linear_group_rope", "group", "rope"] and not st.fused
    log.clear()
    st(512, 0)  # not tried again
    assert log == ["group", "rope"]


def test_error_of_the_call_propagates_and_keeps_the_fused_entry(monkeypatch):
    log = []
    st = _step(log, monkeypatch, fused_ok=False, fallback_fails=True)
    with pytest.raises(ValueError, match="group: refused"):
        st(512, 0)
    assert st.fused and log == ["llhip_linear_group_rope", "group"]
