"""The split launches' bounded wait, forced from the host.

With a spin limit of 0 the first poll that finds a group member's partial
missing gives up: the launch still runs to its end (every wave exits; its
outputs are wrong) and raises the workspace's watchdog word and the device's
host-mapped one.  Nothing here waits on the GPU without bound."""
import numpy as np
import pytest
import torch

from credit_amd import hip_lib
from credit_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu


def _clear():
    try:
        hip_lib.check_watchdog()
    except hip_lib.CreditError:
        pass


def test_expired_wait_is_sticky_until_checked(gpu):
    """The launch after a failed one refuses without a synchronisation of
    its own; credit_check_watchdog reports the failure and clears it; the
    same call then runs and matches the READ variant again."""
    name = "softmax_fwd"
    ins = hip_lib.prepare_inputs(name, WORKLOADS[name].make_inputs(64, 65536, seed=3), gpu)
    outs = hip_lib.allocate_outputs(name, ins)
    ref = hip_lib.allocate_outputs(name, ins)
    hip_lib.HIP_LAUNCHERS[name](ins, ref, hip_lib.LaunchConfig("read", 0))
    torch.cuda.synchronize()
    hip_lib.check_watchdog()

    def split():
        hip_lib.HIP_LAUNCHERS[name](ins, outs, hip_lib.LaunchConfig("split", 16))

    try:
        print("forcing an expired split wait (spin limit 0)", flush=True)
        prev = hip_lib.set_spin_limit(0)
        try:
            split()
            torch.cuda.synchronize()
        finally:
            hip_lib.set_spin_limit(prev)
        with pytest.raises(hip_lib.CreditError) as err:
            split()  # refused on the host: nothing is enqueued
        assert err.value.status == -7  # CREDIT_ERR_WATCHDOG
        with pytest.raises(hip_lib.CreditError) as err:
            hip_lib.check_watchdog()
        assert err.value.status == -7  # CREDIT_ERR_WATCHDOG
        split()
        torch.cuda.synchronize()
        hip_lib.check_watchdog()
        np.testing.assert_allclose(outs[0].cpu().numpy(), ref[0].cpu().numpy(),
                                   rtol=1e-5, atol=1e-6)
    finally:
        _clear()
