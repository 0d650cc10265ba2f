"""Test configuration: the repository root on sys.path, the ``gpu`` marker and the package fixture."""
import importlib
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) GPU and the built libhla_s6.so')


@pytest.fixture(scope='session')
def pkg():
    return importlib.import_module('hybrid-latent-attention_amd')


@pytest.fixture(scope='session')
def ops(pkg):
    return pkg.s6_ops


@pytest.fixture(scope='session')
def layer(pkg):
    return pkg.s6_layer
