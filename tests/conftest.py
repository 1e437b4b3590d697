import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm GPU) and libdispec_hip.so")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def hip():
    """The loaded C-ABI library; GPU tests fail loudly if it is missing."""
    from dispec_amd import _lib
    return _lib.lib()


# -- the IPC peer process ----------------------------------------------------------------
# tests/test_gpu_ipc.py hands payloads to a second process on the same GPU.  That process
# is started here, right after collection and before any test has touched the GPU, with
# the "spawn" context (a fresh interpreter), and only when a selected test asks for it.
_IPC_PEER: dict = {}


def pytest_collection_finish(session):
    if not any("ipc_peer" in getattr(item, "fixturenames", ()) for item in session.items):
        return
    import torch
    if torch.cuda.device_count() < 1:       # counts devices without initialising the GPU
        return
    ctx = torch.multiprocessing.get_context("spawn")
    from dispec_amd.transport.ipc import HipIpcTransport
    msg_q, ack_q = HipIpcTransport.make_queues(ctx)
    cmd_q, res_q = ctx.Queue(), ctx.Queue()
    from tests import _ipc_peer
    proc = ctx.Process(target=_ipc_peer.serve, args=(cmd_q, res_q, msg_q, ack_q), daemon=True)
    proc.start()
    _IPC_PEER.update(proc=proc, cmd=cmd_q, res=res_q, msg=msg_q, ack=ack_q)


def pytest_sessionfinish(session, exitstatus):
    proc = _IPC_PEER.get("proc")
    if proc is None:
        return
    _IPC_PEER["cmd"].put(None)
    proc.join(timeout=60)
    if proc.is_alive():
        proc.kill()
        proc.join(timeout=10)


@pytest.fixture(scope="session")
def ipc_peer():
    """(cmd, res, msg, ack) queues of the peer process, or a failure if it was not started."""
    if "proc" not in _IPC_PEER:
        pytest.fail("the IPC peer process was not started (no GPU visible at collection)")
    if not _IPC_PEER["proc"].is_alive():
        pytest.fail("the IPC peer process has exited")
    return _IPC_PEER
