"""GPU parity of GDN state-pool slot gather/scatter vs index_select/index_copy_."""
import pytest
import torch

from muserve_amd import _lib
from muserve_amd.state_pool import StatePool, gdn_ordinal
from oracle import state as ref
from tests.gpu_util import DEV, case

pytestmark = pytest.mark.gpu


def test_gdn_ordinal():
    gdn = [l for l in range(60) if l % 4 != 3]
    assert [gdn_ordinal(l) for l in gdn] == list(range(45))
    with pytest.raises(ValueError):
        gdn_ordinal(3)


def test_gather_update_scatter_bit_exact():
    case("state pool gather/update/scatter, 3 layers x 64 slots")
    g = torch.Generator().manual_seed(105)
    pool = StatePool(num_layers=3, num_slots=64, device=DEV)
    st_cpu = torch.randn(pool.state.shape, generator=g)
    cv_cpu = torch.randn(pool.conv.shape, generator=g).bfloat16()
    pool.state.copy_(st_cpu.to(DEV))
    pool.conv.copy_(cv_cpu.to(DEV))
    slots = torch.randperm(64, generator=g)[:24].to(torch.int32)
    for layer in range(3):
        st, cv = pool.gather(layer, slots.to(DEV))
        assert torch.equal(st.cpu(), ref.gather(st_cpu, layer, slots))
        assert torch.equal(cv.cpu().view(torch.int16),
                           ref.gather(cv_cpu, layer, slots).view(torch.int16))
        st.add_(1.0)
        cv.mul_(2)
        pool.scatter(layer, slots.to(DEV), st, cv)
        ref.scatter(st_cpu, layer, slots, ref.gather(st_cpu, layer, slots) + 1.0)
        ref.scatter(cv_cpu, layer, slots, ref.gather(cv_cpu, layer, slots) * 2)
    assert torch.equal(pool.state.cpu(), st_cpu)
    assert torch.equal(pool.conv.cpu().view(torch.int16), cv_cpu.view(torch.int16))
    pool.check_errors()


def test_bad_slot_is_reported():
    case("state pool bad slot")
    pool = StatePool(num_layers=1, num_slots=4, state_shape=(2, 8), conv_shape=(8, 4), device=DEV)
    st, cv = pool.gather(0, torch.tensor([1, 9], dtype=torch.int32, device=DEV))
    with pytest.raises(_lib.MkvDeviceError, match="state-pool slot"):
        pool.check_errors()
    assert st[1].abs().sum().item() == 0 and cv[1].float().abs().sum().item() == 0
