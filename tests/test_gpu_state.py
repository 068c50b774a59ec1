"""GPU parity of GDN state-pool slot gather/scatter vs index_select/index_copy_,
and of the in-place decode conv (StatePool.conv_decode) vs the float64 oracle:
the shifted state bit-exact, the output within one bf16 ulp plus the fp32
evaluation term 2^-20 x sum_k |w_k p_k| (which matters only where the
output cancels to near zero)."""
import numpy as np
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


@pytest.mark.parametrize("layers,slots_n", [(3, 64), (45, 8)])
def test_reset_zeroes_only_the_given_slots(layers, slots_n):
    """StatePool.reset vs the oracle's zero initial states: the given slots of
    every layer of both pools become zeros, every other byte is unchanged, an
    out-of-pool slot is flagged and skipped."""
    case(f"state pool reset, {layers} layers x {slots_n} slots")
    g = torch.Generator().manual_seed(layers)
    pool = StatePool(num_layers=layers, num_slots=slots_n, device=DEV)
    st_cpu = torch.randn(pool.state.shape, generator=g)
    cv_cpu = torch.randn(pool.conv.shape, generator=g).bfloat16()
    pool.state.copy_(st_cpu.to(DEV))
    pool.conv.copy_(cv_cpu.to(DEV))
    slots = torch.randperm(slots_n, generator=g)[:max(1, slots_n // 3)].to(torch.int32)
    pool.reset(slots.to(DEV))
    torch.cuda.synchronize()
    pool.check_errors()
    ref.reset(st_cpu, slots)
    ref.reset(cv_cpu, slots)
    assert torch.equal(pool.state.cpu().view(torch.int32), st_cpu.view(torch.int32))
    assert torch.equal(pool.conv.cpu().view(torch.int16), cv_cpu.view(torch.int16))
    pool.reset([])  # nothing to do
    pool.reset([slots_n - 1, slots_n + 5])
    with pytest.raises(_lib.MkvDeviceError, match="state-pool slot"):
        pool.check_errors()
    ref.reset(st_cpu, [slots_n - 1, slots_n + 5])
    ref.reset(cv_cpu, [slots_n - 1, slots_n + 5])
    assert torch.equal(pool.state.cpu().view(torch.int32), st_cpu.view(torch.int32))
    assert torch.equal(pool.conv.cpu().view(torch.int16), cv_cpu.view(torch.int16))


@pytest.mark.parametrize("channels,width", [(2048, 4), (1536, 3)])
def test_conv_decode_in_place(channels, width):
    case(f"GDN decode conv in place, {channels} channels, state width {width}")
    g = torch.Generator().manual_seed(channels + width)
    S, B = 96, 40
    pool = StatePool(num_layers=2, num_slots=S, conv_shape=(channels, width), device=DEV)
    cv_cpu = torch.randn(pool.conv.shape, generator=g).bfloat16()
    pool.conv.copy_(cv_cpu.to(DEV))
    slots = torch.randperm(S, generator=g)[:B].to(torch.int32)
    x = torch.randn(B, channels, generator=g).bfloat16()
    w = (0.6 * torch.randn(channels, 1, 4, generator=g)).bfloat16()
    for step in range(3):  # consecutive steps chain through the slots
        xs = (x * (step + 1)).bfloat16()
        out = pool.conv_decode(1, slots.to(DEV), xs.to(DEV), w.to(DEV))
        torch.cuda.synchronize()
        pool.check_errors()
        p = torch.cat([cv_cpu[1, slots.long(), :, width - 3:].double(),
                       xs.double().unsqueeze(2)], dim=2)
        mass = (w.view(channels, 4).double().unsqueeze(0) * p).abs().sum(2).numpy()
        want = ref.conv_decode(cv_cpu[1], slots, xs, w.view(channels, 4))
        err = (out.cpu().double() - want).abs().numpy()
        mag = np.maximum(np.abs(want.numpy()), 2.0 ** -126)
        tol = 2.0 ** (np.floor(np.log2(mag)) - 7) + 2.0 ** -20 * mass
        assert (err <= tol).all(), f"step {step}: worst {err.max()}"
        assert torch.equal(pool.conv.cpu(), cv_cpu), f"step {step}: state differs"


def test_conv_decode_bad_slot():
    case("GDN decode conv, slot outside the pool")
    pool = StatePool(num_layers=1, num_slots=8, device=DEV)
    pool.conv.normal_()
    before = pool.conv.clone()
    x = torch.randn(2, 2048, device=DEV).bfloat16()
    w = torch.randn(2048, 1, 4, device=DEV).bfloat16()
    out = pool.conv_decode(0, torch.tensor([3, 8], device=DEV), x, w)
    with pytest.raises(_lib.MkvDeviceError, match="state-pool slot out of range"):
        pool.check_errors()
    assert torch.count_nonzero(out[1]) == 0
    assert torch.equal(pool.conv[0, 3, :, :3], before[0, 3, :, 1:])
    keep = [i for i in range(8) if i != 3]
    assert torch.equal(pool.conv[0, keep], before[0, keep])


@pytest.mark.parametrize("width", [4, 3])
def test_decode_gather_equals_gather_plus_conv(width):
    case(f"GDN decode gather (recurrent gather + conv in one launch), width {width}")
    g = torch.Generator().manual_seed(40 + width)
    S, B, C = 64, 24, 2048 if width == 4 else 1536
    a = StatePool(num_layers=2, num_slots=S, conv_shape=(C, width), device=DEV)
    a.state.copy_(torch.randn(a.state.shape, generator=g).to(DEV))
    a.conv.copy_(torch.randn(a.conv.shape, generator=g).bfloat16().to(DEV))
    b = StatePool(num_layers=2, num_slots=S, conv_shape=(C, width), device=DEV)
    b.state.copy_(a.state)
    b.conv.copy_(a.conv)
    slots = torch.randperm(S, generator=g)[:B].to(torch.int32).to(DEV)
    x = torch.randn(B, C, generator=g).bfloat16().to(DEV)
    w = torch.randn(C, 1, 4, generator=g).bfloat16().to(DEV)
    st, out = a.decode_gather(1, slots, x, w)
    st2, _ = b.gather(1, slots, out=(torch.empty_like(st), None))
    out2 = b.conv_decode(1, slots, x, w)
    torch.cuda.synchronize()
    a.check_errors()
    b.check_errors()
    assert torch.equal(st, st2) and torch.equal(st.cpu(), a.state[1, slots.long()].cpu())
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(a.conv, b.conv) and torch.equal(a.state, b.state)
