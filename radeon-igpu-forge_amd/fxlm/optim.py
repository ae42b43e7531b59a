"""fxlm.optim: FlatAdamW -- fp32 flat master + bf16 params + dynamic loss scale.

Surface of ml/fxlm/optim.py:50-196.  At construction every parameter is copied
into one flat fp32 master buffer (each parameter at an 8-element-aligned
offset); m/v are fp32 and a flat bf16 buffer holds the parameters the model
computes with (``p.data`` becomes a view of it).  ``step()`` is one C-ABI call
(fx_adamw_step): sum of squares -> found_inf / grad norm / clip / step counter
/ loss-scale update -> flat AdamW with the bf16 write-back.  No host sync and
no host-to-device copy.
"""
import ctypes

import torch

from fxgpu.abi import MAX_TENSORS, call, fxAdamWState, fxTensorList, lib, stream_of


def _align8(n):
    return (n + 7) & ~7


class FlatAdamW:
    """fp32 master + bf16 params + dynamic loss scaling + global grad clipping.

    opt = FlatAdamW(model, lr=3e-4, betas=(0.9,0.95), eps=1e-8,
                    weight_decay=0.1, max_grad_norm=1.0,
                    init_scale=2.**16, growth_interval=1000)
    opt.backward(loss)              # (loss * opt.scale).backward()
    stats = opt.step(lr=...)        # {grad_norm, found_inf, scale}: 0-dim cuda tensors
    opt.zero_grad()                 # set_to_none
    """

    def __init__(self, model, lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1,
                 max_grad_norm=1.0, init_scale=2.0 ** 16, growth_interval=1000):
        named = [(n, p) for n, p in model.named_parameters() if p.requires_grad]
        if not named:
            raise ValueError("model has no parameter with requires_grad")
        dev = named[0][1].device
        if dev.type != "cuda":
            raise TypeError("parameters must be cuda tensors")
        if any(p.dtype != torch.float32 for _n, p in named):
            raise TypeError("FlatAdamW expects fp32 parameters (it builds the bf16 copy)")
        self.lr, self.betas, self.eps = lr, betas, eps
        self.weight_decay, self.max_grad_norm = weight_decay, max_grad_norm
        self.growth_interval = int(growth_interval)

        self._info = []     # (name, p, off, numel, wd_flag)
        total = 0
        for name, p in named:
            self._info.append((name, p, total, p.numel(),
                               1 if (p.dim() >= 2 and weight_decay != 0) else 0))
            total += _align8(p.numel())
        self.numel = total
        self.master = torch.zeros(total, device=dev, dtype=torch.float32)
        self.m = torch.zeros(total, device=dev, dtype=torch.float32)
        self.v = torch.zeros(total, device=dev, dtype=torch.float32)
        self.flat16 = torch.zeros(total, device=dev, dtype=torch.bfloat16)
        for _name, p, off, n, _wd in self._info:
            self.master[off:off + n] = p.data.reshape(-1)
        self.flat16.copy_(self.master)
        for _name, p, off, n, _wd in self._info:
            p.data = self.flat16[off:off + n].view(p.shape)

        self._step_ctr = torch.zeros((), device=dev, dtype=torch.int32)
        self._found_inf = torch.zeros((), device=dev, dtype=torch.float32)
        self._norm = torch.zeros((), device=dev, dtype=torch.float32)
        self.scale = torch.full((), float(init_scale), device=dev, dtype=torch.float32)
        self._growth = torch.zeros((), device=dev, dtype=torch.int32)
        self._work = torch.empty(0, device=dev, dtype=torch.float32)

    # -- helpers -------------------------------------------------------------

    def _lists(self):
        """Tensor lists (<= 64 entries each) over the parameters that have a gradient."""
        items = []
        for name, p, off, n, wd in self._info:
            g = p.grad
            if g is None:
                continue
            if g.dtype != torch.bfloat16:
                raise TypeError(f"{name}: gradient must be bfloat16 ({g.dtype})")
            if not g.is_contiguous():
                g = g.contiguous()
            if g.data_ptr() % 16:
                raise RuntimeError(f"{name}: gradient is not 16-byte aligned")
            items.append((g, off, n, wd))
        lists = (fxTensorList * max(1, (len(items) + MAX_TENSORS - 1) // MAX_TENSORS))()
        nl = 0
        for i in range(0, len(items), MAX_TENSORS):
            tl = lists[nl]
            chunk = items[i:i + MAX_TENSORS]
            for j, (g, off, n, wd) in enumerate(chunk):
                tl.g[j] = g.data_ptr()
                tl.off[j] = off
                tl.n[j] = n
                tl.wd[j] = wd
            tl.count = len(chunk)
            nl += 1
        return lists, nl, items

    # -- API -------------------------------------------------------------------

    def backward(self, loss):
        (loss * self.scale).backward()

    def step(self, lr=None):
        lr_v = self.lr if lr is None else float(lr)
        lists, nl, _keep = self._lists()   # _keep holds contiguous grad copies alive
        need = lib().fx_adamw_workspace(lists, nl) // 4
        if self._work.numel() < need:
            self._work = torch.empty(need, device=self.master.device, dtype=torch.float32)
        st = self._state(lr_v, self._work.data_ptr())
        call("fx_adamw_step", ctypes.byref(st), lists, nl, stream_of(self.master))
        return {"grad_norm": self._norm, "found_inf": self._found_inf, "scale": self.scale}

    def _state(self, lr_v, work):
        """The fxAdamWState of this optimiser for one step at learning rate lr_v."""
        st = fxAdamWState()
        st.master, st.m, st.v = self.master.data_ptr(), self.m.data_ptr(), self.v.data_ptr()
        st.p16 = self.flat16.data_ptr()
        st.step = self._step_ctr.data_ptr()
        st.found_inf = self._found_inf.data_ptr()
        st.grad_norm = self._norm.data_ptr()
        st.scale = self.scale.data_ptr()
        st.growth = self._growth.data_ptr()
        st.work = work
        st.lr, st.beta1, st.beta2 = lr_v, float(self.betas[0]), float(self.betas[1])
        st.eps, st.weight_decay = float(self.eps), float(self.weight_decay)
        st.max_grad_norm = float(self.max_grad_norm)
        st.growth_factor, st.backoff_factor = 2.0, 0.5
        st.growth_interval = self.growth_interval
        return st

    def zero_grad(self):
        for _n, p, _o, _el, _w in self._info:
            p.grad = None

    # -- state -----------------------------------------------------------------

    def state_dict(self):
        return {"master": self.master, "m": self.m, "v": self.v,
                "step": self._step_ctr, "scale": self.scale, "growth": self._growth,
                "offsets": [(n_, o, el) for n_, _p, o, el, _w in self._info]}

    def load_state_dict(self, sd):
        self.master.copy_(sd["master"])
        self.m.copy_(sd["m"])
        self.v.copy_(sd["v"])
        self._step_ctr.copy_(sd["step"])
        self.scale.copy_(sd["scale"])
        self._growth.copy_(sd["growth"])
        self.flat16.copy_(self.master)     # refresh the bf16 views

    def master_state_dict(self):
        """fp32 master weights under the model's parameter names."""
        return {name: self.master[off:off + n].view(p.shape)
                for name, p, off, n, _w in self._info}
