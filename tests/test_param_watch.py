"""CPU checks of _lib.ParamWatch, the validity test of the caches that hold
values derived from module parameters (the site blocks' bf16 weights and
the detection head's folded parameters): it stays valid while nothing
changes and turns invalid on an in-place update, a reassigned parameter, a
replaced submodule, a dtype move and an updated buffer."""
import torch
import torch.nn as nn

from ssla_amd import _lib


def _net():
    return nn.Sequential(nn.Linear(4, 3), nn.BatchNorm1d(3))


def _watch(net):
    return _lib.ParamWatch(net, ["0.weight", "0.bias", "1.running_mean", "1.weight", "1.num_batches_tracked"])


def test_valid_until_something_changes():
    net = _net()
    w = _watch(net)
    assert w.valid() and w.valid()
    with torch.no_grad():
        net[0].weight.add_(1.0)
    assert not w.valid()


def test_reassigned_parameter_and_replaced_module():
    net = _net()
    w = _watch(net)
    net[0].bias = nn.Parameter(net[0].bias.detach().clone())
    assert not w.valid()
    w = _watch(net)
    net[1] = nn.BatchNorm1d(3)
    assert not w.valid()


def test_buffer_update_and_move():
    net = _net()
    w = _watch(net)
    net.train()
    net(torch.randn(5, 4))   # running statistics and the batch counter updated in place
    assert not w.valid()
    w = _watch(net)
    net.to(torch.float64)
    assert not w.valid()


def test_absent_buffer():
    net = nn.Sequential(nn.BatchNorm1d(3, track_running_stats=False))
    w = _lib.ParamWatch(net, ["0.weight", "0.num_batches_tracked"])
    assert w.valid()
    with torch.no_grad():
        net[0].weight.mul_(2.0)
    assert not w.valid()
