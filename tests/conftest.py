import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU through the qmm C-ABI library")


def _reload_qmm_tuning_on_change():
    """libqmm reads its QMM_* overrides once (a launch never reads the environment) and re-reads them
    at qmm_reload_tuning(). Tests force kernel choices by changing those variables through os.environ
    (monkeypatch.setenv / delenv included), which goes through os.putenv / os.unsetenv: wrap both so
    that every change of a QMM_* variable is followed by a reload in the library, when it is loaded."""
    put, unset = os.putenv, os.unsetenv

    def reload_if_qmm(key):
        k = key.decode() if isinstance(key, bytes) else key
        if not k.startswith("QMM_"):
            return
        mod = sys.modules.get("inference_amd.qmm")
        if mod is not None and mod._lib is not None:
            mod._lib.qmm_reload_tuning()

    def putenv(key, value):
        put(key, value)
        reload_if_qmm(key)

    def unsetenv(key):
        unset(key)
        reload_if_qmm(key)

    os.putenv, os.unsetenv = putenv, unsetenv


_reload_qmm_tuning_on_change()
