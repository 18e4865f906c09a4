"""Compile a Lowered program with hipRTC and run it as one cooperative launch.

Mirrors the reference's ``vesta/launch.py`` surface (``TORCH_DT``,
``compile_code`` in place of ``compile_cubin`` :17-27, ``Kernel`` :29-73 with
``view``/``bind``/``launch``/``__call__``), over the repository's own native
shim ``libvesta_hip.so`` (C ABI in include/vesta_hip.h) instead of NVRTC and
the CUDA driver. torch supplies the device buffers and the stream; the shim
owns only module and function handles.

There is no fallback: if the shim is not built or no GPU is present, the
calls that need them raise.
"""
from __future__ import annotations

import atexit
import ctypes
import hashlib
import os
import sys
import threading
import weakref

LIB_DIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), '_lib')
LIB_PATH = os.path.join(LIB_DIR, 'libvesta_hip.so')
CACHE_DIR = os.environ.get('VESTA_CACHE', os.path.join(os.path.dirname(os.path.abspath(__file__)), '_cache'))
ARCH = os.environ.get('VESTA_ARCH', 'gfx950')
# Packed fp32 vector ops stay off (they have given silent wrong results on
# these parts); -O3 for the generated kernel.
RTC_OPTS = ('-O3', '-std=c++17', '-ffp-contract=off',
            '-mllvm', '-amdgpu-early-inline-all=true',
            '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops')

# Profiling only: issue the persistent kernels with an ordinary launch
# (vh_launch) instead of a cooperative one, for runs under rocprofv3, whose
# own teardown has ended in a segmentation fault after every run that made
# cooperative launches. The kernel is the same; its grid barriers still need
# every block resident, which holds on an otherwise idle device (the grid is
# at most one block per CU, checked at construction). Were a block not
# resident, the barrier's bounded wait would set error code 1 and every
# block would exit, so the launch ends either way; check() then raises.
PLAIN_LAUNCH = os.environ.get('VESTA_PLAIN_LAUNCH', '') == '1'

_lib = None
_lib_lock = threading.Lock()


def lib():
    """The loaded shim (ctypes.CDLL). Raises if it has not been built."""
    global _lib
    with _lib_lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(f'{LIB_PATH} is missing: build it with __graft_entry__.build()')
            L = ctypes.CDLL(LIB_PATH)
            vp, sz, ip, cp = ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int), ctypes.c_char_p
            sig = {
                'vh_compile': [cp, cp, ctypes.POINTER(cp), ctypes.c_int, ctypes.POINTER(vp), ctypes.POINTER(sz),
                               ctypes.POINTER(vp)],
                'vh_module_load': [vp, ctypes.POINTER(vp)],
                'vh_module_get_function': [vp, cp, ctypes.POINTER(vp)],
                'vh_module_unload': [vp],
                'vh_function_set_dynamic_lds': [vp, ctypes.c_int],
                'vh_function_attrs': [vp, ip, ip, ip, ip],
                'vh_occupancy': [vp, ctypes.c_int, sz, ip],
                'vh_device_info': [ctypes.c_int, ip, ip, ip, cp, sz],
                'vh_launch_cooperative': [vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp, ctypes.POINTER(vp)],
                'vh_launch': [vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp, ctypes.POINTER(vp)],
                'vh_noalloc_scratch': [ctypes.POINTER(vp), ctypes.POINTER(sz)],
                'vh_noalloc_layout': [sz, sz, sz, ctypes.POINTER(sz), ctypes.POINTER(sz)],
                'vh_noalloc_read': [vp, sz, sz, vp],
                'vh_launch_cooperative_noalloc': [vp, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, vp,
                                                  ctypes.POINTER(vp), ctypes.c_int, ctypes.c_int, sz, sz, sz],
                'vh_synchronize': [],
            }
            for name, args in sig.items():
                fn = getattr(L, name)
                fn.argtypes, fn.restype = args, ctypes.c_int
            L.vh_free.argtypes, L.vh_free.restype = [vp], None
            L.vh_error_string.argtypes, L.vh_error_string.restype = [ctypes.c_int], ctypes.c_char_p
            _lib = L
        return _lib


# Objects holding a loaded module. They are unloaded by an exit hook, which
# runs while the interpreter and the HIP runtime are whole; left to garbage
# collection at interpreter shutdown, a module can outlive the runtime's own
# teardown (and a profiler's finalisation, which then sees a code object it
# has already forgotten).
_live = weakref.WeakSet()
_hook = []


def track(owner):
    """Register ``owner`` (it has ``close()``) for unloading at exit."""
    _live.add(owner)
    if not _hook:
        atexit.register(_close_all)
        _hook.append(True)


def _close_all():
    for owner in list(_live):
        try:
            owner.close()
        except Exception:
            pass


def unload(module_handle):
    """Wait for the device, then unload a module (skipped once the interpreter
    is shutting down: the exit hook has already unloaded what it could)."""
    if sys.is_finalizing():
        return
    lib().vh_synchronize()                  # no launch of this module may still be running
    lib().vh_module_unload(module_handle)


def ok(status, what=''):
    if status != 0:
        msg = lib().vh_error_string(status).decode(errors='replace')
        raise RuntimeError(f'{what}: {msg} (status {status})' if what else f'{msg} (status {status})')


ROCM_DIR = os.path.realpath(os.environ.get('ROCM_PATH', '/opt/rocm'))


def rtc_version() -> str:
    """The ROCm release whose hipRTC compiles the kernels (the image's own)."""
    try:
        with open(os.path.join(ROCM_DIR, '.info', 'version')) as fh:
            return fh.read().strip()
    except OSError:
        return 'unknown'


def _rtc_in_process() -> bool:
    """Is the hipRTC this process has mapped the image's own? torch ships its
    own hipRTC and compiler (an older ROCm, which allocates registers
    differently); once torch is loaded first, the shim binds to that copy."""
    L = lib()
    del L
    try:
        with open('/proc/self/maps') as fh:
            paths = {ln.split()[-1] for ln in fh if 'libhiprtc' in ln or 'libamd_comgr' in ln}
    except OSError:
        return 'torch' not in sys.modules
    return all(os.path.realpath(p).startswith(ROCM_DIR + os.sep) for p in paths)


def _compile_here(src: str, full) -> bytes:
    L = lib()
    arr = (ctypes.c_char_p * len(full))(*[o.encode() for o in full])
    code, size, log = ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_void_p()
    st = L.vh_compile(src.encode(), b'vesta_step.hip', arr, len(full), ctypes.byref(code), ctypes.byref(size),
                      ctypes.byref(log))
    text = ctypes.string_at(log.value).decode(errors='replace') if log.value else ''
    if log.value:
        L.vh_free(log)
    if st != 0:
        raise RuntimeError(f'hipRTC failed ({L.vh_error_string(st).decode()}):\n{text}')
    blob = ctypes.string_at(code.value, size.value)
    L.vh_free(code)
    return blob


def _compile_file(src_path: str, out_path: str, full) -> None:
    """Child-process side of ``compile_code``: no torch loaded, so the shim's
    hipRTC is the image's."""
    with open(src_path) as fh:
        src = fh.read()
    try:
        blob = _compile_here(src, list(full))
    except RuntimeError as e:
        sys.stderr.write(str(e))
        sys.exit(3)
    with open(out_path, 'wb') as fh:
        fh.write(blob)


def _compile_child(src: str, full) -> bytes:
    import subprocess
    import tempfile
    pkg = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    with tempfile.TemporaryDirectory(prefix='vesta_rtc_') as d:
        sp, op = os.path.join(d, 'k.hip'), os.path.join(d, 'k.co')
        with open(sp, 'w') as fh:
            fh.write(src)
        code = (f'import sys; sys.path.insert(0, {pkg!r}); from vesta import launch; '
                f'launch._compile_file({sp!r}, {op!r}, {list(full)!r})')
        r = subprocess.run([sys.executable, '-c', code], capture_output=True, text=True)
        if r.returncode == 3:
            raise RuntimeError(r.stderr)
        if r.returncode != 0 or not os.path.exists(op):
            raise RuntimeError(f'the hipRTC compile process failed (status {r.returncode}):\n{r.stderr[-4000:]}')
        with open(op, 'rb') as fh:
            return fh.read()


def compile_code(src: str, arch: str = ARCH, opts=RTC_OPTS, cache: bool = True) -> bytes:
    """HIP C++ -> gfx950 code object through hipRTC (replaces NVRTC, reference
    launch.py:17-27). Failures raise RuntimeError carrying the compile log.
    Always the image's ROCm hipRTC: in a process where torch's copy is the one
    mapped, the compile runs in a child process. Code objects are cached on
    disk by a hash of source, arch, options and that ROCm release."""
    full = [f'--offload-arch={arch}', *opts]
    key = hashlib.sha256((src + '\0' + '\0'.join(full) + '\0rocm ' + rtc_version()).encode()).hexdigest()[:32]
    path = os.path.join(CACHE_DIR, key + '.co')
    if cache and os.path.exists(path):
        with open(path, 'rb') as fh:
            return fh.read()
    blob = _compile_here(src, full) if _rtc_in_process() else _compile_child(src, full)
    if cache:
        os.makedirs(CACHE_DIR, exist_ok=True)
        tmp = f'{path}.{os.getpid()}.tmp'
        with open(tmp, 'wb') as fh:
            fh.write(blob)
        os.replace(tmp, path)
    return blob


PREFETCH_BUDGETS = (64, 24, 16)   # registers per lane a site may prefetch into, tried in turn (B=8, which
                                  # spills at 64, with a 384-position cache: 308-310 us per step at 16-28,
                                  # 320 at 32, 337 at 48; with 448 positions 24 and 32 are even)
PREFETCH_BUDGETS_PACKED = (24, 16)   # ... the same from 4 to 8 rows (same box, four models each built
                                     # alternately, 24 against 64: small at 8 rows 285.3 / 289.4 us per step, at 4
                                     # rows 255.5 / 257.8, medium at 8 rows 730.9 / 735.1; 16 and 28 at 8 rows
                                     # 290.5 / 290.2; at one row 64 stays, 195.0 against 200.2)
SPILLS_OK = 4                     # spilled registers a kernel may keep (outside its hot loops; GPT-2 small
                                  # B=8, same box: 298.5 us per step with 8 spilled at the first try, 296.2
                                  # with 1 at the next)


def code_spills(code: bytes) -> int:
    """The ``.vgpr_spill_count`` recorded in a code object's kernel metadata
    (a MessagePack map: the key string, then an unsigned integer)."""
    key = b'.vgpr_spill_count'
    i = code.find(key)
    if i < 0:
        return 0
    j = i + len(key)
    b = code[j]
    if b <= 0x7f:
        return b
    width = {0xcc: 1, 0xcd: 2, 0xce: 4, 0xcf: 8}.get(b)
    return int.from_bytes(code[j + 1:j + 1 + width], 'big') if width else 0


def lower_fitted(lower_fn, text, res, **kw):
    """``lower_fn(text, res, **kw)`` with the largest prefetch register budget
    (of PREFETCH_BUDGETS, or PREFETCH_BUDGETS_PACKED from 4 to 8 rows),
    and at it the deepest unprefetched MFMA pipeline (``MFMA_PIPES``), whose
    kernel spills at most SPILLS_OK registers (compiling each try; the code
    objects are cached, so the chosen one is not compiled again)."""
    from .mfma import MFMA_PIPES, MFMA_ROWS_MIN
    budgets = PREFETCH_BUDGETS_PACKED if MFMA_ROWS_MIN <= kw.get('batch', 1) <= 8 else PREFETCH_BUDGETS
    tries = [(b, d) for b in budgets for d in MFMA_PIPES]
    for budget, pipe in tries:
        low = lower_fn(text, res, prefetch_vgprs=budget, mfma_pipe=pipe, **kw)
        if (budget, pipe) == tries[-1] or code_spills(compile_code(low.src)) <= SPILLS_OK:
            return low


def device_info(dev: int = 0) -> dict:
    cu, coop, lds = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    arch = ctypes.create_string_buffer(128)
    ok(lib().vh_device_info(dev, ctypes.byref(cu), ctypes.byref(coop), ctypes.byref(lds), arch, 128), 'device info')
    return dict(cu_count=cu.value, cooperative=bool(coop.value), lds_per_block=lds.value, arch=arch.value.decode())


def _torch():
    import torch
    return torch


def torch_dtypes():
    torch = _torch()
    return {'f32': torch.float32, 'f16': torch.float16, 'i32': torch.int32}


class _LazyDT(dict):
    def __missing__(self, k):
        self.update(torch_dtypes())
        return dict.__getitem__(self, k)


TORCH_DT = _LazyDT()


REFERENCE_BLOCK = 256        # the reference's default threads per block (reference launch.py:30)


def resolve_block(block, lowered_block):
    """The block a generated kernel runs with: its own (``lowered_block``) for
    ``None`` or the reference default, else ``block`` if it is that one."""
    if block in (None, REFERENCE_BLOCK):
        return lowered_block
    if block != lowered_block:
        raise ValueError(f'kernel was lowered for {lowered_block} threads per block, not {block}')
    return block


class Kernel:
    """One generated kernel, loaded on the current device and launched
    cooperatively on torch's current stream (reference launch.py:29-73).

    ``block``: the generated kernel fixes its own block (``lowered.block``,
    eight waves of 64); the reference default 256 (eight 32-wide warps) and
    ``None`` mean that block, any other value is an error.

    grid = blocks that fit per CU (occupancy at the block and the
    kernel's LDS, at most the lowering's ``per_cu_max``) x CUs, optionally
    capped by ``blocks_per_sm`` and by the lowering's own grid limit. ``S`` (fp32 scratch), ``bar`` (barrier and
    reduction counters, zeroed once; the kernel leaves them zeroed) and ``TS``
    (timing sums) are allocated here.

    A grid barrier that waits too long (only a launch whose blocks are not all
    resident can get there) gives up and raises an error word in ``bar``;
    ``check()`` reads it (one device synchronisation) and raises.
    """

    def __init__(self, lowered, block=REFERENCE_BLOCK, device=0, blocks_per_sm=None):
        torch = _torch()
        if not torch.cuda.is_available():
            raise RuntimeError('no GPU: the Vesta kernel needs a ROCm device')
        torch.cuda.set_device(device)
        torch.zeros(1, device='cuda')                       # make torch's context current
        self.device = device
        self.info = device_info(device)
        if not self.info['cooperative']:
            raise RuntimeError('device does not support cooperative launch')
        block = resolve_block(block, lowered.block)
        self.code = compile_code(lowered.src)
        L = lib()
        mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
        ok(L.vh_module_load(self.code, ctypes.byref(mod)), 'module load')
        self.mod = mod
        track(self)
        ok(L.vh_module_get_function(mod, lowered.name.encode(), ctypes.byref(fn)), 'get function')
        self.fn = fn
        self.smem = lowered.shared_bytes
        if self.smem > 65536:       # up to 64 KB needs no opt-in
            ok(L.vh_function_set_dynamic_lds(fn, self.smem), 'dynamic LDS')
        per = ctypes.c_int()
        ok(L.vh_occupancy(fn, block, self.smem, ctypes.byref(per)), 'occupancy')
        per_cu = min(per.value, lowered.per_cu_max)
        if blocks_per_sm:
            per_cu = min(per_cu, blocks_per_sm)
        self.per_cu = per_cu
        self.cus = self.info['cu_count']
        if per_cu * self.cus < lowered.grid_max:
            raise RuntimeError(f'the kernel is laid out for {lowered.grid_max} resident blocks; this device holds '
                               f'{per_cu} per CU x {self.cus} CUs')
        if PLAIN_LAUNCH and lowered.grid_max > self.cus:
            raise RuntimeError(f'VESTA_PLAIN_LAUNCH needs at most one block per CU: {lowered.grid_max} blocks, '
                               f'{self.cus} CUs')
        self.grid = lowered.grid_max
        self.block = block
        regs, slds, priv, mxb = (ctypes.c_int() for _ in range(4))
        ok(L.vh_function_attrs(fn, ctypes.byref(regs), ctypes.byref(slds), ctypes.byref(priv), ctypes.byref(mxb)),
           'function attributes')
        self.attrs = dict(regs=regs.value, static_lds=slds.value, private_bytes=priv.value, max_block=mxb.value)
        self.lowered = lowered
        self.S = torch.zeros(max(1, lowered.scratch_floats), dtype=torch.float32, device='cuda')
        self.bar = torch.zeros(lowered.counters, dtype=torch.int32, device='cuda')
        # timing: clock ticks per (site, block), site-major
        # and, after it, each block's arrival / release time at the barriers of a launch's last step
        from .lower import BTRACE
        self.TS = torch.zeros(max(1024, (len(lowered.sites) + 2 * BTRACE) * self.grid), dtype=torch.int64,
                              device='cuda')
        self.args = None

    def view(self, name):
        """A torch view of a value kept in global scratch (no copy, no sync)."""
        off, _, shape = self.lowered.scratch[name]
        n = 1
        for s in shape:
            n *= s
        return self.S[off:off + max(1, n)].view(*shape) if shape else self.S[off]

    def bind(self, residue):
        """Fix the argument list once; a launch is then one shim call. Residues
        the kernel reads through a transposed copy are copied here: bind again
        after changing them."""
        vals = []
        self._packed = {}
        for name, dt, _ in self.lowered.params:
            if name in self.lowered.packs:
                # a copy of a read-only residue transposed in its last two axes (made once, here)
                t = residue[self.lowered.packs[name]].transpose(-1, -2).contiguous()
                self._packed[name] = t
            else:
                t = residue[name]
            if not (t.is_cuda and t.dtype == TORCH_DT[dt] and t.is_contiguous()):
                raise TypeError(f'residue {name}: need a contiguous {dt} device tensor, got {t.dtype} '
                                f'{"device" if t.is_cuda else "host"} {"contiguous" if t.is_contiguous() else "strided"}')
            want = self.lowered.shapes[name]
            if tuple(t.shape) != tuple(want) and not (want == () and t.numel() == 1):
                raise ValueError(f'residue {name}: shape {tuple(t.shape)} but the kernel was lowered for {want}')
            vals.append(t.data_ptr())
        vals += [self.S.data_ptr(), self.bar.data_ptr(), self.TS.data_ptr()]
        self._slots = [ctypes.c_void_p(v) for v in vals]
        self._nsteps = ctypes.c_int(1)
        self._tok = ctypes.c_void_p(0)
        self._tok_in = ctypes.c_void_p(0)
        ptrs = [ctypes.cast(ctypes.pointer(x), ctypes.c_void_p) for x in self._slots]
        ptrs += [ctypes.cast(ctypes.pointer(v), ctypes.c_void_p) for v in (self._nsteps, self._tok, self._tok_in)]
        self.args = (ctypes.c_void_p * len(ptrs))(*ptrs)
        self.keep = residue

    def _steps_and_tokens(self, steps, tokens, inputs, what):
        """Host checks shared by ``launch`` and ``launch_noalloc``, made before
        anything is enqueued: the kernel writes ``steps * history`` chosen
        tokens into ``tokens`` and reads as many inputs from ``inputs``, so
        both must be contiguous int32 tensors on this kernel's device holding
        at least that many elements."""
        if self.args is None:
            raise RuntimeError(f'bind() the residues before {what}()')
        steps = int(steps)
        if steps < 1:
            raise ValueError('steps must be at least 1')
        need = steps * int(getattr(self.lowered, 'history', 0) or 0)
        ptrs = []
        for arg, t in (('tokens', tokens), ('inputs', inputs)):
            if t is None:
                ptrs.append(0)
                continue
            if not need:
                raise ValueError(f'{arg}: {self.lowered.name} records no tokens (no token feedback)')
            if not (getattr(t, 'is_cuda', False) and t.dtype == TORCH_DT['i32'] and t.is_contiguous()):
                raise TypeError(f'{arg} must be a contiguous int32 device tensor')
            if t.device.index is not None and t.device.index != self.device:
                raise ValueError(f'{arg} is on device {t.device.index}; the kernel runs on device {self.device}')
            if t.numel() < need:
                raise ValueError(f'{arg} holds {t.numel()} tokens; {steps} steps of {need // steps} rows need {need}')
            ptrs.append(t.data_ptr())
        self._nsteps.value = steps
        self._tok.value, self._tok_in.value = ptrs

    def launch(self, steps=1, tokens=None, inputs=None):
        """Run ``steps`` steps in one cooperative launch on torch's current
        stream (no sync). With token feedback, ``tokens`` (int32 device tensor,
        at least steps * B elements) receives each step's chosen tokens, and
        ``inputs`` (int32 device tensor [steps, B]) forces the input of steps
        1..steps-1 (the first step reads the residue as usual)."""
        self._steps_and_tokens(steps, tokens, inputs, 'launch')
        stream = _torch().cuda.current_stream().cuda_stream
        if PLAIN_LAUNCH:
            ok(lib().vh_launch(self.fn, self.grid, self.block, self.smem, ctypes.c_void_p(stream), self.args),
               'launch (VESTA_PLAIN_LAUNCH, profiling)')
        else:
            ok(lib().vh_launch_cooperative(self.fn, self.grid, self.block, self.smem, ctypes.c_void_p(stream),
                                           self.args), 'cooperative launch')
        self._noalloc_bar = None

    def __call__(self, residue):
        self.bind(residue)
        self.launch()

    def launch_noalloc(self, steps=1, tokens=None, inputs=None):
        """``launch`` through ``vh_launch_cooperative_noalloc``: S, bar and TS
        are the library's static per-device scratch instead of this object's
        buffers (nothing is allocated; outputs left in S are read with
        ``read_noalloc``). Calls on one device share that scratch. The error
        word of such a launch is in the static scratch's barrier block:
        ``check()`` reads it there."""
        self._steps_and_tokens(steps, tokens, inputs, 'launch_noalloc')
        if PLAIN_LAUNCH:
            raise RuntimeError('launch_noalloc is cooperative only (unset VESTA_PLAIN_LAUNCH)')
        sizes = (self.S.numel() * 4, self.bar.numel() * 4, self.TS.numel() * 8)
        bar_off, ts_off = ctypes.c_size_t(), ctypes.c_size_t()
        ok(lib().vh_noalloc_layout(*sizes, ctypes.byref(bar_off), ctypes.byref(ts_off)), 'static scratch layout')
        stream = _torch().cuda.current_stream().cuda_stream
        ok(lib().vh_launch_cooperative_noalloc(self.fn, self.grid, self.block, self.smem, ctypes.c_void_p(stream),
                                               self.args, len(self.args), len(self.lowered.params), *sizes),
           'cooperative launch (static scratch)')
        self._noalloc_bar = bar_off.value

    def read_noalloc(self, name, out):
        """Copy value ``name`` (a scratch value, e.g. 'logit') from the static
        scratch into the fp32 device tensor ``out`` (on the current stream)."""
        off, _, shape = self.lowered.scratch[name]
        n = 1
        for d in shape:
            n *= d
        if not (out.is_cuda and out.dtype == TORCH_DT['f32'] and out.is_contiguous() and out.numel() == max(1, n)):
            raise TypeError(f'out must be a contiguous fp32 device tensor of {max(1, n)} values')
        stream = _torch().cuda.current_stream().cuda_stream
        ok(lib().vh_noalloc_read(ctypes.c_void_p(out.data_ptr()), off * 4, out.numel() * 4, ctypes.c_void_p(stream)),
           'static scratch read')

    def _error_word(self):
        """The error word of the last launch (one device synchronisation):
        from this object's ``bar``, or from the static scratch's barrier block
        when the last launch was ``launch_noalloc``."""
        from .lower import BAR_ERROR
        bar_off = getattr(self, '_noalloc_bar', None)
        if bar_off is None:
            return int(self.bar[BAR_ERROR].item()) if self.bar.numel() > BAR_ERROR else 0
        word = self._noalloc_word()
        stream = _torch().cuda.current_stream().cuda_stream
        ok(lib().vh_noalloc_read(ctypes.c_void_p(word.data_ptr()), bar_off + 4 * BAR_ERROR, 4,
                                 ctypes.c_void_p(stream)), 'static scratch read')
        return int(word.item())

    def _noalloc_word(self):
        w = getattr(self, '_noalloc_word_t', None)
        if w is None:
            w = self._noalloc_word_t = _torch().zeros(1, dtype=_torch().int32, device=self.bar.device)
        return w

    def check(self):
        """Raise if a grid barrier of an earlier launch gave up waiting (reads
        the error word: one device synchronisation). The barrier words are
        cleared first, so the kernel can be launched again (the static
        scratch of ``launch_noalloc`` is cleared by its next call)."""
        from .lower import ERR_BARRIER, ERR_RANGE
        code = self._error_word()
        if code:
            self.bar.zero_()
            self._noalloc_bar = None
            why = {ERR_BARRIER: f'a grid barrier gave up waiting (are all {self.grid} blocks resident on the '
                                f'device?)',
                   ERR_RANGE: 'an activation beyond the fp16 range (65504) reached a matrix-core product'}
            raise RuntimeError(f'{self.lowered.name}: {why.get(code, f"error word {code}")}; the launch\'s results '
                               f'are invalid')

    def close(self):
        if getattr(self, 'mod', None) is not None and self.mod.value:
            try:
                unload(self.mod)
            finally:
                self.mod = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
