"""CPU-side checks of the PyTorch custom operators and of the drop-in's import seam (no kernel launches):
every operator is registered under torch.ops.yoco_z1 with the mutation annotations it needs; the shard update traces
into a graph of those operators on fake tensors (what torch.compile sees); CPU tensors are refused; ``import
faster_yoco_amd`` works from the repository root; and importing zero1_fast with YOCO_ZERO1_FAST=1 installs the patches
on fairseq's mixin (and on the reference's layer_graphs / CEReduce seams) as yoco/tasks/zero1_fast.py:247-255 does,
checked against stand-in modules placed in sys.modules."""
import os
import subprocess
import sys
import textwrap

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# operator -> the arguments it writes (the schema must say so, and say nothing else)
MUTATES = {
    'grad_sumsq_': {'partials'}, 'norm_clip_': {'factor', 'norm', 'grad_norm'},
    'grad_norm_clip_': {'partials', 'factor', 'norm', 'grad_norm'},
    'update_scalars_': {'factor', 'norm', 'grad_norm', 'flags', 'clip_log'},
    'grad_update_scalars_': {'partials', 'factor', 'norm', 'grad_norm', 'flags', 'clip_log'},
    'clip_factor_': {'factor', 'grad_norm'}, 'adam_cast_': {'p', 'm', 'v', 'p16'},
    'adam_cast_gout_': {'p', 'm', 'v', 'p16', 'g32'},
    'adam_cast_dev_': {'p', 'm', 'v', 'p16'}, 'bias_corrections_step_': {'step', 'bc'},
    'owner_sum_': {'out', 'out_sum', 'partials'},
    'owner_sum_update_': {'out', 'workspace', 'out_sum', 'factor', 'norm', 'grad_norm', 'flags', 'clip_log'},
    'sum_slots_': {'out', 'waves'}, 'reduce_waves_': {'partials'}, 'scale_up_': {'g32'}, 'cast_bf16_': {'p16'},
    'embedding_dense_backward_out_': {'out', 'workspace'}, 'embedding_dense_backward': {'workspace'},
}


def test_every_operator_is_registered_with_its_mutations(pkg):
    from faster_yoco_amd import library
    assert set(library.OPS) == set(MUTATES)
    for name, writes in MUTATES.items():
        schema = getattr(torch.ops.yoco_z1, name).default._schema
        mutable = {a.name for a in schema.arguments if a.alias_info is not None and a.alias_info.is_write}
        assert mutable == writes, (name, mutable)
        assert bool(schema.returns) == (name == 'embedding_dense_backward')


def test_shard_update_traces_to_operators_on_fake_tensors(pkg):
    """The update a caller compiles -- norm + clip chain, device step counter, Adam + BF16 -- traced with fake
    tensors: every launch is a yoco_z1 operator node, nothing falls out of the graph."""
    from torch._subclasses.fake_tensor import FakeTensorMode
    from torch.fx.experimental.proxy_tensor import make_fx
    import faster_yoco_amd.library  # noqa: F401
    ops = torch.ops.yoco_z1

    def update(g, p, m, v, p16, partials, factor, grad_norm, step, bc):
        ops.grad_norm_clip_(1234, [g], partials, factor, None, grad_norm, 1.0, None)
        ops.bias_corrections_step_(step, bc, 0.9, 0.95, 1)
        ops.adam_cast_dev_(1234, [g], [p], [m], [v], [p16], factor, bc, 3e-4, 0.9, 0.95, 1e-8, 0.1, 1)
        return grad_norm

    with FakeTensorMode():
        f32 = lambda n: torch.empty(n, device='cuda')
        args = (f32(4096), f32(4096), f32(4096), f32(4096), torch.empty(4096, dtype=torch.bfloat16, device='cuda'),
                torch.empty(2048, dtype=torch.float64, device='cuda'), f32(1), f32(1),
                torch.empty(1, dtype=torch.int64, device='cuda'), f32(2))
        gm = make_fx(update, tracing_mode='fake')(*args)
    called = [str(n.target) for n in gm.graph.nodes if n.op == 'call_function']
    assert called == ['yoco_z1.grad_norm_clip_.default', 'yoco_z1.bias_corrections_step_.default',
                      'yoco_z1.adam_cast_dev_.default']


def test_shard_update_functionalizes_on_fake_tensors(pkg):
    """The same update through AOT autograd on fake tensors (the functionalization torch.compile applies): every
    mutating operator is wrapped functionally (auto_functionalized) and the graph keeps all of them."""
    from torch._functorch.aot_autograd import aot_function
    from torch._subclasses.fake_tensor import FakeTensorMode
    import faster_yoco_amd.library  # noqa: F401
    ops = torch.ops.yoco_z1

    def update(g, p, m, v, p16, partials, factor, grad_norm, step, bc):
        ops.grad_norm_clip_(1234, [g], partials, factor, None, grad_norm, 1.0, 1.0)
        ops.bias_corrections_step_(step, bc, 0.9, 0.95, 1)
        ops.adam_cast_dev_(1234, [g], [p], [m], [v], [p16], factor, bc, 3e-4, 0.9, 0.95, 1e-8, 0.1, 1)
        ops.adam_cast_(1234, [g], [p], [m], [v], [p16], factor, 3e-4, 0.9, 0.95, 1e-8, 0.5, 0.5, 0.1, 1, 0, 1)
        ops.owner_sum_update_([p16, p16], p16.clone(), partials, 0.5, None, factor, None, grad_norm, None, None,
                              None, 1.0, 1.0, None)
        return grad_norm

    graphs = []

    def keep(gm, example_inputs):
        graphs.append(gm)
        return gm

    with FakeTensorMode():
        f32 = lambda n: torch.empty(n, device='cuda')
        args = (f32(4096), f32(4096), f32(4096), f32(4096), torch.empty(4096, dtype=torch.bfloat16, device='cuda'),
                torch.empty(4096, dtype=torch.float64, device='cuda'), f32(1), f32(1),
                torch.empty(1, dtype=torch.int64, device='cuda'), f32(2))
        aot_function(update, fw_compiler=keep)(*args)
    text = str(graphs[0].graph)
    for name in ('grad_norm_clip_', 'bias_corrections_step_', 'adam_cast_dev_', 'adam_cast_.default',
                 'owner_sum_update_'):
        assert f'yoco_z1.{name}' in text, name
    assert 'auto_functionalized' in text


def test_operators_refuse_cpu_tensors(pkg):
    import faster_yoco_amd.library  # noqa: F401
    ops = torch.ops.yoco_z1
    t = torch.zeros(8)
    with pytest.raises(RuntimeError, match='no CPU path'):
        ops.cast_bf16_(t, torch.zeros(8, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match='no CPU path'):
        ops.norm_clip_(torch.zeros(2048, dtype=torch.float64), None, None, None, 1.0, 1.0)
    with pytest.raises(RuntimeError, match='no CPU path'):
        ops.embedding_dense_backward(torch.zeros(4, 2, dtype=torch.bfloat16), torch.zeros(4, dtype=torch.int64), 5,
                                     -1, 1.0, 0, torch.zeros(64, dtype=torch.uint8))


def test_operator_library_host_entry_points(pkg):
    """libyoco_z1_torch.so is bound to the C ABI library and registers tables with checked arguments (no device
    work: a registered handle is only recorded)."""
    import ctypes
    from faster_yoco_amd import _lib, library
    L = library.OPS_LIB
    assert L.z1t_init(_lib.lib()._name.encode()) == 0
    assert L.z1t_init(b'/nonexistent/libyoco_z1.so') == -1            # not a loaded library: refused
    assert L.z1t_init(_lib.lib()._name.encode()) == 0                  # bound again to the right one
    rows = (_lib.Z1Tensor * 2)(_lib.Z1Tensor(None, None, None, None, None, 10),
                               _lib.Z1Tensor(None, None, None, None, None, 6))
    fake = ctypes.c_void_p(0x1000)
    assert L.z1t_table_register(None, 0, 0, 0, 2, rows, None) == -1   # no table
    assert L.z1t_table_register(fake, 0, 7, 0, 2, rows, None) == -1   # unknown gradient dtype
    assert L.z1t_table_register(fake, 0, 0, 0, -1, rows, None) == -1  # negative row count
    bad = (ctypes.c_int64 * 2)(0, -4)
    assert L.z1t_table_register(fake, 0, 0, 0, 2, rows, bad) == -1    # negative flat offset
    offs = (ctypes.c_int64 * 2)(0, 16)
    assert L.z1t_table_register(fake, 0, 0, 0, 2, rows, offs) == 0
    L.z1t_table_forget(fake)
    L.z1t_table_forget(fake)                                           # forgetting twice is harmless


def _run(script, env_extra, prelude=''):
    env = dict(os.environ)
    for k in list(env):
        if k.startswith('YOCO_'):
            del env[k]
    env.update(env_extra)
    code = textwrap.dedent(prelude) + textwrap.dedent(script)
    res = subprocess.run([sys.executable, '-c', code], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=240)
    assert res.returncode == 0, res.stdout + res.stderr
    return res.stdout.strip().splitlines()[-1]


STAND_INS = '''
    import sys, types
    def module(name, **attrs):
        m = types.ModuleType(name)
        m.__dict__.update(attrs)
        sys.modules[name] = m
        return m
    class _FP16OptimizerMixin:
        def clip_grad_norm(self, max_norm, aggregate_norm_fn=None): pass
        def step(self, closure=None, groups=None): pass
        def zero_grad(self): pass
    module('fairseq'); module('fairseq.optim')
    module('fairseq.optim.fp16_optimizer', _FP16OptimizerMixin=_FP16OptimizerMixin)
    ddp_calls = []
    class CEReduce:
        def _sum(self, ph): pass
    module('models'); module('models.decoder')
    module('models.decoder.layer_graphs', PRE_DDP_HOOKS=[], install_ddp_patch=lambda: ddp_calls.append(1))
    module('models.decoder.ce_reduce', CEReduce=CEReduce)
'''


def test_package_imports_under_its_python_name(pkg):
    out = _run('''
        import faster_yoco_amd, os
        from faster_yoco_amd import zero1_fast, ops
        print(faster_yoco_amd.__name__, os.path.basename(faster_yoco_amd.__path__[0]), zero1_fast.__name__)
    ''', {})
    assert out == 'faster_yoco_amd faster-yoco_amd faster_yoco_amd.zero1_fast'


def test_zero1_fast_installs_at_import_with_the_switch(pkg):
    out = _run('''
        import faster_yoco_amd.zero1_fast as z
        lg = sys.modules['models.decoder.layer_graphs']
        from faster_yoco_amd import ce_reduce
        print(_FP16OptimizerMixin.clip_grad_norm is z.clip_grad_norm, _FP16OptimizerMixin.step is z.step,
              _FP16OptimizerMixin.zero_grad is z.zero_grad, lg.PRE_DDP_HOOKS == [z._place_params], ddp_calls == [1],
              CEReduce._sum is ce_reduce._sum, sorted(z.INSTALLED), z.FOLD_SCALE)
    ''', {'YOCO_ZERO1_FAST': '1', 'YOCO_ZERO1_ALLGATHER': '1', 'YOCO_ZERO1_PARAM_VIEWS': '1', 'YOCO_CE_REDUCE': '1'},
               STAND_INS)
    assert out == "True True True True True True ['ce_reduce', 'fp16_optimizer', 'layer_graphs'] False"


def test_zero1_fast_leaves_fairseq_alone_without_the_switch(pkg):
    out = _run('''
        orig = _FP16OptimizerMixin.step
        import faster_yoco_amd.zero1_fast as z
        print(_FP16OptimizerMixin.step is orig, z.INSTALLED, sys.modules['models.decoder.layer_graphs'].PRE_DDP_HOOKS)
    ''', {}, STAND_INS)
    assert out == 'True [] []'


def test_zero1_fast_imports_without_fairseq(pkg):
    out = _run('''
        import faster_yoco_amd.zero1_fast as z
        print(z.ENABLED, z.INSTALLED)
    ''', {'YOCO_ZERO1_FAST': '1'})
    assert out == 'True []'
