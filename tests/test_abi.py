"""The C-ABI library loads and exports every entry point include/anehip.h
declares.  CPU-only: no compute call is made."""
import subprocess

import pytest


def test_library_exports_every_declared_symbol(anehip_mod):
    L = anehip_mod.lib()
    declared = anehip_mod.declared_symbols()
    assert len(declared) >= 10
    missing = [s for s in declared if not hasattr(L, s)]
    assert not missing, f"declared but not exported: {missing}"


def test_exports_are_c_abi(anehip_mod):
    out = subprocess.run(["nm", "-D", "--defined-only", anehip_mod.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    names = {l.split()[-1] for l in out.splitlines() if " T " in l}
    for s in anehip_mod.declared_symbols():
        assert s in names, f"{s} is not an unmangled exported function"


def test_init_reports_status_without_crashing(anehip_mod):
    rc = anehip_mod.lib().anehip_init()
    assert rc in (0, -8)  # ANEHIP_OK or ANEHIP_ENODEV
    if rc != 0:
        assert anehip_mod.lib().anehip_last_error(None)


def test_ctx_create_rejects_null_out(anehip_mod):
    rc = anehip_mod.lib().anehip_ctx_create(0, None, None)
    assert rc == -1
    assert b"out is NULL" in anehip_mod.lib().anehip_last_error(None)
