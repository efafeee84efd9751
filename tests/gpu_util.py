"""Helpers for GPU tests: device tensors and mr_epilogue descriptors from Python."""
import numpy as np

from mira_amd import _lib as L


def dev():
    import torch
    return torch.device("cuda:0")


def T(a: np.ndarray):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev())


def empty(shape, dtype):
    import torch
    return torch.zeros(shape, dtype=dtype, device=dev())


def stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream


def sync():
    import torch
    torch.cuda.synchronize()


def epilogue(steps=(), scale=None, out_f32=None, ldo=0, out_i8=None, ldq=0, xs=1.0, out_acc=None, ldacc=0,
             keep=None):
    """steps: (fn name, mode, operand tensor or None, ld, swapped)."""
    e = L.Epilogue()
    e.n_steps = len(steps)
    for i, (fn, mode, t, ld, sw) in enumerate(steps):
        e.steps[i].fn = L.EPI_FN[fn]
        e.steps[i].mode = mode
        e.steps[i].ptr = t.data_ptr() if t is not None else None
        e.steps[i].ld = ld
        e.steps[i].swapped = int(sw)
    e.scale = scale.data_ptr() if scale is not None else None
    e.out_f32 = out_f32.data_ptr() if out_f32 is not None else None
    e.ldo = ldo
    e.out_i8 = out_i8.data_ptr() if out_i8 is not None else None
    e.ldq = ldq
    e.out_xs = xs
    e.out_acc = out_acc.data_ptr() if out_acc is not None else None
    e.ldacc = ldacc
    return e


def oracle_env(g, feeds: dict) -> dict:
    """Every value of a graph evaluated by the oracle, keyed by ir.Value."""
    from oracle import golden as G
    env = {v: np.asarray(feeds[v.name]).astype(v.type.np_dtype) for v in g.inputs}
    for op in g.ops:
        if op.is_control:
            env.update(zip(op.results, G.control(op, [env[x] for x in op.inputs])))
        else:
            env[op.result] = G.evaluate(op.kind, [env[x] for x in op.inputs], op.attrs)
    return env
