"""@newt.autotune / @newt.heuristics (reference newt/runtime/autotuner.py:5-128).

Same protocol as the reference: each config is timed with do_bench, configs
that fail to compile or launch are skipped, the fastest is cached per key
(values of the `key` arguments, shapes for tensors, plus every tensor's dtype),
`reset_to_zero` arguments are zeroed before every timed run and once more
before the real launch after tuning. Configs that would need more LDS than
gfx950 has fail at compile time and are skipped like any invalid config.
"""


class Config:
    def __init__(self, kwargs, num_warps=4, num_stages=1):
        self.kwargs = dict(kwargs)
        self.num_warps = num_warps
        self.num_stages = num_stages

    def all_kwargs(self):
        return {**self.kwargs, "num_warps": self.num_warps, "num_stages": self.num_stages}

    def __repr__(self):
        kw = ", ".join(f"{k}={v}" for k, v in self.kwargs.items())
        return f"Config({kw}, num_warps={self.num_warps})"


class Autotuner:
    def __init__(self, jitfn, configs, key, reset_to_zero=None, warmup=5, rep=20):
        self.jitfn = jitfn
        self.configs = configs
        self.key = key
        self.reset_to_zero = reset_to_zero or []
        self.warmup = warmup
        self.rep = rep
        self.cache = {}
        self.best_config = None
        self.timings = {}
        self.__name__ = getattr(jitfn, "__name__", "kernel")
        self.param_names = getattr(jitfn, "param_names", [])
        self.defaults = getattr(jitfn, "defaults", {})

    def __getitem__(self, grid):
        def runner(*args, **kwargs):
            return self._run(grid, args, kwargs)

        return runner

    def _key_values(self, args, kwargs):
        import torch

        bound = dict(zip(self.jitfn.param_names, args))
        bound.update(kwargs)
        for n, d in getattr(self.jitfn, "defaults", {}).items():
            bound.setdefault(n, d)
        vals = []
        for k in self.key:
            v = bound.get(k)
            vals.append(tuple(v.shape) if hasattr(v, "shape") else v)
        for v in bound.values():
            if isinstance(v, torch.Tensor):
                vals.append(str(v.dtype))
        return tuple(vals)

    def _run(self, grid, args, kwargs):
        from ..testing import do_bench

        keyv = self._key_values(args, kwargs)
        bound = dict(zip(self.jitfn.param_names, args))
        bound.update(kwargs)
        best = self.cache.get(keyv)
        tuned_now = False
        if best is None:
            tuned_now = True
            timings = []
            last_exc = None
            for cfg in self.configs:
                call_kwargs = {**kwargs, **cfg.kwargs, "num_warps": cfg.num_warps,
                               "num_stages": cfg.num_stages}

                def run_cfg(call_kwargs=call_kwargs):
                    for name in self.reset_to_zero:
                        bound[name].zero_()
                    self.jitfn[grid](*args, **call_kwargs)

                try:
                    ms = do_bench(run_cfg, warmup=self.warmup, rep=self.rep)
                    timings.append((ms, cfg))
                except Exception as e:  # invalid config (LDS, tiling, ...)
                    last_exc = e
                    continue
            if not timings:
                raise RuntimeError(f"autotune: no valid config for {self.__name__}") from last_exc
            timings.sort(key=lambda t: t[0])
            self.timings[keyv] = timings
            best = timings[0][1]
            self.cache[keyv] = best
        self.best_config = best
        if tuned_now:
            for name in self.reset_to_zero:
                bound[name].zero_()
        self.jitfn[grid](*args, **{**kwargs, **best.kwargs, "num_warps": best.num_warps,
                                   "num_stages": best.num_stages})


def autotune(configs, key, reset_to_zero=None):
    def deco(jitfn):
        return Autotuner(jitfn, configs, key, reset_to_zero)

    return deco


class Heuristics:
    def __init__(self, jitfn, values):
        self.jitfn = jitfn
        self.values = values
        self.__name__ = getattr(jitfn, "__name__", "kernel")
        self.param_names = jitfn.param_names
        self.defaults = getattr(jitfn, "defaults", {})

    def __getitem__(self, grid):
        def runner(*args, **kwargs):
            bound = dict(zip(self.jitfn.param_names, args))
            bound.update(kwargs)
            for name, fn in self.values.items():
                kwargs[name] = fn(bound)
            return self.jitfn[grid](*args, **kwargs)

        return runner


def heuristics(values):
    def deco(jitfn):
        return Heuristics(jitfn, values)

    return deco
