"""Engine: the kernel primitives of the prefill pass, on gfx950 HIP kernels.

This mirrors the primitive surface of the reference Engine
(quail/backends/quail/executor/attention.py:432-562, 1235-1275): norm_quant,
gemm, qk_norm_rope, attention, activation_quant, quant, fused_add_rms_norm,
write_kv and kv_row_scatter, with the same arguments, return values and
in-place updates, so a pipeline written against the reference Engine runs
unchanged. Every primitive launches hand-written kernels of
libquail_mi355x.so through its C ABI on torch's current stream; tensors are
torch-allocated (the library allocates nothing). There is no CPU or
PyTorch fallback: without the native library the primitives raise.

Layouts are the reference's: FP8 activations are e4m3fn (n, K) with
"column-major" fp32 scales, a (K/128, n) tensor viewed as (n, K/128)
(attention.py:534-537); weights are e4m3 (N, K) with weight_scale_inv
(N/128, K/128).
"""

import os

import torch

from quail_amd import _lib

GROUP = 128

# GEMM tile configurations (csrc/gemm_fp8.hip), in two arithmetic families.
# Promotion family (30, 31): each 128-K block's products summed from zero by
# one 16x16x128 MFMA and promoted into an fp32 total, total += (sA * sW) *
# partial (DeepGEMM's form), persistent grids; 30 = 256 tokens x 256
# weights, 31 = 256 x 320 (widths that are multiples of 320: whole waves
# where N = 2560 makes 2.5 or 1.25 waves of 256 x 256 tiles). Rescale family
# (10, 11, 12, 22): the MFMA accumulators rescaled in place by s_prev / s at
# each block; 10 = 256 x 256, one workgroup per tile; 11 = 256 x 128 (widths
# not a multiple of 256); 22 = config 10's tiles on a persistent grid; 12 =
# 256 x 320. Within a family every config computes each output element with
# the same operations in the same order, so the choice among them never
# changes a bit. The family is a function of N alone, so a row's result
# never depends on how many rows share the launch (a document packed with
# others equals itself run alone, bit for bit): N a multiple of 256 or 320
# takes the promotion family, the rest config 11. QUAIL_GEMM_CONFIG forces
# one.
GEMM_CONFIG_ENV = "QUAIL_GEMM_CONFIG"
GEMM_CONFIGS = (10, 11, 12, 22, 30, 31)
RESCALE_CONFIGS = (10, 11, 12, 22)
PROMOTION_CONFIGS = (30, 31)
GEMM_PROMOTION_CONFIG = 30
GEMM_PROMOTION_WIDE_CONFIG = 31
SWIGLU_DEFAULT_CONFIG = 30
GEMM_ODD_WIDTH_CONFIG = 11
CUS = 256


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def gemm_config(n: int, k: int, m: int) -> int:
    """The tile configuration of an (m x k) by (n x k) GEMM: the promotion
    family for widths that are a multiple of 256 or 320 (256 x 320 tiles
    where they take fewer full-wave units, or where 256 x 256 ones cannot
    tile N), config 11 for the rest."""
    forced = os.environ.get(GEMM_CONFIG_ENV)
    if forced is not None:
        return int(forced)
    if n % 256 == 0 or n % 320 == 0:
        if n % 320 == 0 and (n % 256 or _wide_tiles_fill_better(n, m)):
            return GEMM_PROMOTION_WIDE_CONFIG
        return GEMM_PROMOTION_CONFIG
    return GEMM_ODD_WIDTH_CONFIG


def _wave_cost(tiles: int) -> float:
    """Time of `tiles` equal tiles on the CUs, in full-wave units: a partial
    last wave of fraction f costs about 0.5 + 0.5 f of a full one (its tiles
    run faster with fewer neighbours sharing the loads; measured ~0.75 at f
    = 0.5 on the N = 2560 shapes)."""
    full, rest = divmod(tiles, CUS)
    return full + (0.5 + 0.5 * rest / CUS if rest else 0.0)


def _wide_tiles_fill_better(n: int, m: int) -> bool:
    """256 x 320 tiles (1.25x the work of 256 x 256) take fewer full-wave
    units: N = 2560 at M = 8192 (256 tiles against 320) or a 16k-row pack
    (512 against 640)."""
    tm = -(-m // 256)
    return 1.25 * _wave_cost(tm * (n // 320)) < (_wave_cost(tm * (n // 256)) if n % 256 == 0
                                                 else float("inf"))


SWIGLU_CONFIG_ENV = "QUAIL_SWIGLU_CONFIG"


def swiglu_config(n: int = 0, k: int = 0, m: int = 0) -> int:
    """Tile schedule of the gate_up GEMM with the SiLU-quant epilogue (n =
    gate_up rows, 256 per tile): the promotion kernel (30) for every shape;
    10 and 22 (the rescale family) stay selectable. QUAIL_SWIGLU_CONFIG
    forces it alone, QUAIL_GEMM_CONFIG with every GEMM."""
    for env in (SWIGLU_CONFIG_ENV, GEMM_CONFIG_ENV):
        forced = os.environ.get(env)
        if forced is not None and int(forced) in (10, 22, 30):
            return int(forced)
    return SWIGLU_DEFAULT_CONFIG


class Engine:
    """Kernels, quantization and paged attention over the KV arena.

    Args:
        arena: KVArena the attention path reads and writes.
        num_q_heads, num_kv_heads, head_dim: attention geometry.
        rotary: the model's rotary module (its `cos_sin_cache`).
        fp8: whether the linear weights are fp8 block-quantized; this engine
            runs FP8 checkpoints only.
        kernels: "quail" or "vllm" (accepted for interface parity; both
            select the fused HIP kernels).
    """

    def __init__(self, arena, *, num_q_heads, num_kv_heads, head_dim, rotary, fp8=True,
                 kernels="quail"):
        if kernels not in ("quail", "vllm"):
            raise ValueError(f"kernels must be 'quail' or 'vllm', got {kernels!r}")
        if not fp8:
            raise ValueError("this engine runs FP8 block-quantized checkpoints only")
        lib = _lib.load()
        if lib.qx_device_is_gfx950() != 1:
            raise RuntimeError("the quail_amd engine needs a gfx950 (MI350/MI355X) device")
        self.kernels = kernels
        self.torch = torch
        self.arena = arena
        self.rotary = rotary
        self.num_q_heads = num_q_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.fp8 = torch.float8_e4m3fn
        self.is_fp8 = True
        self.use_ue8m0 = False
        # a list to receive (M, N, K, start event, end event, SwiGLU epilogue)
        # per timed GEMM launch, recorded on the launch stream; None (the
        # default) records nothing. A timed launch costs the stream two event
        # records (each leaves the GPU idle a few microseconds), so one launch
        # in gemm_timer_every is timed; gemm_launches counts them all
        self.gemm_timer = None
        self.gemm_timer_every = 1
        self.gemm_launches = 0

    # ---- weights and quant --------------------------------------------

    @staticmethod
    def weight_scale(linear):
        for name in ("weight_scale", "weight_scale_inv"):
            scale = getattr(linear, name, None)
            if scale is not None:
                return scale
        raise AttributeError(f"no weight scale on {type(linear).__name__}")

    def _col_major_scales(self, num_tokens, width, device="cuda"):
        return torch.empty((width // GROUP, num_tokens), dtype=torch.float32,
                           device=device).permute(1, 0)

    @staticmethod
    def _scale_ld(scales):
        # a (tokens, groups) view of (groups, tokens) storage: group stride
        return scales.stride(1) if scales.dim() == 2 else scales.shape[0]

    def gemm(self, q_input, input_scale, linear, out=None):
        """bf16 q_input @ W^T with the FP8 block scales applied per 128 of K."""
        w = linear.weight
        sw = self.weight_scale(linear)
        m, k = q_input.shape
        n = w.shape[0]
        if w.shape[1] != k:
            raise ValueError(f"gemm: input width {k} vs weight {tuple(w.shape)}")
        if input_scale.shape != (m, k // GROUP) or input_scale.stride(0) != 1:
            raise ValueError("gemm: activation scales must be the (tokens, K/128) view of "
                             "column-major storage")
        if out is None:
            out = torch.empty((m, n), dtype=torch.bfloat16, device=q_input.device)
        timed = self._timed_launch()
        if timed:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
        _lib.call("qx_gemm_fp8_blockscaled", _ptr(q_input), _ptr(input_scale), _ptr(w),
                  _ptr(sw), _ptr(out), m, n, k, q_input.stride(0), out.stride(0),
                  self._scale_ld(input_scale), gemm_config(n, k, m), _stream())
        if timed:
            end.record()
            self.gemm_timer.append((m, n, k, start, end, False))
        return out

    def _timed_launch(self):
        """Whether this GEMM launch is timed: gemm_timer is set and the launch
        is the first of its gemm_timer_every."""
        if self.gemm_timer is None:
            return False
        self.gemm_launches += 1
        return (self.gemm_launches - 1) % self.gemm_timer_every == 0

    def gate_up_activation_quant(self, q_input, input_scale, linear):
        """The gate_up projection and the quantized SiLU-gated product in one
        launch: `activation_quant(gemm(q_input, input_scale, linear))`
        (qwen3.py:66-67), bit for bit, without writing the bf16 gate_up rows.
        `linear` is the checkpoint's gate_up projection as it is."""
        w = linear.weight
        sw = self.weight_scale(linear)
        m, k = q_input.shape
        n = w.shape[0]
        if w.shape[1] != k:
            raise ValueError(f"gate_up: input width {k} vs weight {tuple(w.shape)}")
        if n % 256:
            raise ValueError(f"gate_up: width {n} is not a multiple of 256")
        if input_scale.shape != (m, k // GROUP) or input_scale.stride(0) != 1:
            raise ValueError("gate_up: activation scales must be the (tokens, K/128) view of "
                             "column-major storage")
        half = n // 2
        q = torch.empty((m, half), dtype=self.fp8, device=q_input.device)
        scales = self._col_major_scales(m, half, q_input.device)
        timed = self._timed_launch()
        if timed:
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
        _lib.call("qx_gemm_fp8_swiglu_quant", _ptr(q_input), _ptr(input_scale), _ptr(w),
                  _ptr(sw), _ptr(q), q.stride(0), _ptr(scales), self._scale_ld(scales), m, half,
                  k, q_input.stride(0), self._scale_ld(input_scale), swiglu_config(n, k, m),
                  _stream())
        if timed:
            end.record()
            self.gemm_timer.append((m, n, k, start, end, True))
        return q, scales

    def quant(self, x, *, output=None):
        """Per-token 128-group FP8 of bf16 rows: (e4m3 rows, col-major scales)."""
        n, k = x.shape
        if output is not None:
            q, scales = output
        else:
            q = torch.empty((n, k), dtype=self.fp8, device=x.device)
            scales = self._col_major_scales(n, k, x.device)
        _lib.call("qx_group_quant", _ptr(x), x.stride(0), _ptr(q), q.stride(0), _ptr(scales),
                  self._scale_ld(scales), n, k, _stream())
        return q, scales

    def rms_norm(self, x, norm):
        return self.norm_rows(x, norm.weight, norm.variance_epsilon)

    def norm_rows(self, x, weight, eps):
        """vLLM rms_norm of the last dimension: bf16(bf16(x * rstd) * w)."""
        width = x.shape[-1]
        rows = x.reshape(-1, width)
        if not rows.is_contiguous():
            rows = rows.contiguous()
        out = torch.empty_like(rows)
        # z = x + 0 leaves x; the residual copy goes to a scratch row set
        zeros = torch.zeros_like(rows)
        _lib.call("qx_add_rmsnorm", _ptr(rows), rows.stride(0), _ptr(zeros), zeros.stride(0),
                  None, _ptr(weight), _ptr(out), out.stride(0), None, 0, rows.shape[0],
                  width, float(eps), _stream())
        return out.view(x.shape)

    def fused_add_rms_norm(self, hidden, residual, norm):
        """In place, as vLLM: residual <- bf16(hidden + residual);
        hidden <- rms_norm(residual). Returns (hidden, residual)."""
        n, h = hidden.shape
        _lib.call("qx_add_rmsnorm", _ptr(hidden), hidden.stride(0), _ptr(residual),
                  residual.stride(0), None, _ptr(norm.weight), _ptr(hidden), hidden.stride(0),
                  _ptr(residual), residual.stride(0), n, h, float(norm.variance_epsilon),
                  _stream())
        return hidden, residual

    def final_norm(self, hidden, residual, final_indices, norm):
        """fused_add_rms_norm of the rows final_indices selects, gathered in
        the same kernel (qwen3.py:130-134); returns the normed rows."""
        rows = final_indices.shape[0]
        h = hidden.shape[1]
        out = torch.empty((rows, h), dtype=torch.bfloat16, device=hidden.device)
        _lib.call("qx_add_rmsnorm", _ptr(hidden), hidden.stride(0), _ptr(residual),
                  residual.stride(0), _ptr(final_indices), _ptr(norm.weight), _ptr(out),
                  out.stride(0), None, 0, rows, h, float(norm.variance_epsilon), _stream())
        return out

    # ---- the primitives a forward loop calls ---------------------------

    def norm_quant(self, hidden, norm, residual=None):
        """RMS-normed, quantized GEMM input; adds the residual first when given."""
        n, h = hidden.shape
        q = torch.empty((n, h), dtype=self.fp8, device=hidden.device)
        scales = self._col_major_scales(n, h, hidden.device)
        eps = float(norm.variance_epsilon)
        if residual is None:
            _lib.call("qx_rmsnorm_quant", _ptr(hidden), hidden.stride(0), _ptr(norm.weight),
                      _ptr(q), q.stride(0), _ptr(scales), self._scale_ld(scales), n, h, eps,
                      _stream())
        else:
            _lib.call("qx_add_rmsnorm_quant", _ptr(hidden), hidden.stride(0), _ptr(residual),
                      residual.stride(0), _ptr(norm.weight), _ptr(q), q.stride(0), _ptr(scales),
                      self._scale_ld(scales), n, h, eps, _stream())
        return q, scales

    def embed_norm_quant(self, ids, embed_weight, norm):
        """Embedding gather fused with layer 0's norm_quant: returns
        (q, scales, residual) where residual holds the embedded rows."""
        n = ids.shape[0]
        h = embed_weight.shape[1]
        residual = torch.empty((n, h), dtype=torch.bfloat16, device=ids.device)
        q = torch.empty((n, h), dtype=self.fp8, device=ids.device)
        scales = self._col_major_scales(n, h, ids.device)
        _lib.call("qx_embed_rmsnorm_quant", _ptr(embed_weight), embed_weight.stride(0),
                  _ptr(ids), _ptr(residual), residual.stride(0), _ptr(norm.weight), _ptr(q),
                  q.stride(0), _ptr(scales), self._scale_ld(scales), n, h,
                  float(norm.variance_epsilon), _stream())
        return q, scales, residual

    def activation_quant(self, gate_up):
        """SiLU-gated product of the two gate_up halves, quantized."""
        n, doubled = gate_up.shape
        half = doubled // 2
        q = torch.empty((n, half), dtype=self.fp8, device=gate_up.device)
        scales = self._col_major_scales(n, half, gate_up.device)
        _lib.call("qx_silu_mul_quant", _ptr(gate_up), gate_up.stride(0), _ptr(q), q.stride(0),
                  _ptr(scales), self._scale_ld(scales), n, half, _stream())
        return q, scales

    def _rope_cache(self):
        cache = self.rotary.cos_sin_cache
        if cache.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError(f"cos_sin_cache dtype {cache.dtype}")
        if cache.shape[1] != self.head_dim:
            raise ValueError(f"cos_sin_cache width {cache.shape[1]} != head_dim {self.head_dim}")
        return cache

    def qk_norm_rope(self, qkv, positions, attn):
        """Per-head normed and rotated q and k from the fused qkv output."""
        n = qkv.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        q = torch.empty((n, hq * d), dtype=torch.bfloat16, device=qkv.device)
        k = torch.empty((n, hk * d), dtype=torch.bfloat16, device=qkv.device)
        cache = self._rope_cache()
        _lib.call("qx_qk_norm_rope", _ptr(qkv), qkv.stride(0), _ptr(q), q.stride(0), _ptr(k),
                  k.stride(0), _ptr(cache), int(cache.dtype == torch.float32), _ptr(positions),
                  _ptr(attn.q_norm.weight), _ptr(attn.k_norm.weight), n, hq, hk, d,
                  float(attn.q_norm.variance_epsilon), _stream())
        return q, k

    def qk_norm_rope_rows(self, qkv, positions, attn, identity=None, meta=None):
        """q, k and v rows in one pass over qkv (qx_qk_norm_rope_kv with the
        identity row map; `identity` = arange(n) int64 on the device, made
        here when not given): the tree path's call A reads K and V of the
        pack's own rows contiguous, V of the arena's V type. With a tree
        pack's meta carrying `row_pool_dst` (pool row
        per pack row, -1 for none), the same pass also writes the pack's KV
        into the arena pages of meta's layer (the kv_src -> kv_dst writes,
        attention.py:1405)."""
        n = qkv.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        if qkv.shape[1] < (hq + 2 * hk) * d:
            raise ValueError(f"qkv width {qkv.shape[1]} < {(hq + 2 * hk) * d}")
        dev = qkv.device
        q = torch.empty((n, hq * d), dtype=torch.bfloat16, device=dev)
        k = torch.empty((n, hk * d), dtype=torch.bfloat16, device=dev)
        v_dtype = self._v_dtype()
        v = torch.empty((n, hk * d), dtype=v_dtype, device=dev)
        rows = identity if identity is not None else torch.arange(n, dtype=torch.int64,
                                                                   device=dev)
        if rows.shape[0] != n or rows.dtype != torch.int64:
            raise ValueError("identity must be arange(n) int64")
        cache = self._rope_cache()
        pools, dst2 = (None, None), None
        if meta is not None and meta.get("row_pool_dst") is not None:
            dst2 = meta["row_pool_dst"]
            if dst2.shape[0] != n:
                raise ValueError(f"row_pool_dst has {dst2.shape[0]} rows, qkv {n}")
            pools = self.arena.layer_kv(meta["layer"])
            self._check_pools(*pools)
        _lib.call("qx_qk_norm_rope_kv", _ptr(qkv), qkv.stride(0), _ptr(q), q.stride(0), _ptr(k),
                  _ptr(v), _ptr(rows), _ptr(pools[0]), _ptr(pools[1]), _ptr(dst2), _ptr(cache),
                  int(cache.dtype == torch.float32),
                  _ptr(positions), _ptr(attn.q_norm.weight), _ptr(attn.k_norm.weight), n, hq,
                  hk, d, float(attn.q_norm.variance_epsilon), int(v_dtype == torch.float16),
                  _stream())
        if dst2 is not None:
            meta["kv_fresh_layer"] = meta["layer"]
        return q, k, v

    def qk_norm_rope_kv(self, qkv, positions, attn, meta):
        """qk_norm_rope that also writes every row's K and V into the arena
        pages of meta's layer (pool row meta["unified"]["row_dst"][i]; the
        fresh-row write of write_kv, attention.py:1178-1191, in the same pass
        over qkv). Returns q; this layer's write_kv then copies only the
        retained tails."""
        n = qkv.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        if qkv.shape[1] < (hq + 2 * hk) * d:
            raise ValueError(f"qkv width {qkv.shape[1]} < {(hq + 2 * hk) * d}")
        dst = meta["unified"]["row_dst"]
        if dst.shape[0] != n:
            raise ValueError(f"row_dst has {dst.shape[0]} rows, qkv {n}")
        layer = meta["layer"]
        k_pool, v_pool = self.arena.layer_kv(layer)
        self._check_pools(k_pool, v_pool)
        q = torch.empty((n, hq * d), dtype=torch.bfloat16, device=qkv.device)
        cache = self._rope_cache()
        _lib.call("qx_qk_norm_rope_kv", _ptr(qkv), qkv.stride(0), _ptr(q), q.stride(0),
                  _ptr(k_pool), _ptr(v_pool), _ptr(dst), None, None, None, _ptr(cache),
                  int(cache.dtype == torch.float32), _ptr(positions), _ptr(attn.q_norm.weight),
                  _ptr(attn.k_norm.weight), n, hq, hk, d, float(attn.q_norm.variance_epsilon),
                  int(v_pool.dtype == torch.float16), _stream())
        meta["kv_fresh_layer"] = layer
        return q

    def kv_norm_rope(self, qkv, positions, attn, meta):
        """The K/V half of qk_norm_rope_kv: every row's normed, rotated K and
        its V go into the arena pages of meta's layer, and q stays as the
        projection left it; this layer's paged attention then normalizes and
        rotates q as it loads it (qx_paged_attention_qnorm), with the same
        arithmetic (bit for bit). Returns the raw q columns of qkv (a view)."""
        n = qkv.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        if d != GROUP or qkv.shape[1] < (hq + 2 * hk) * d:
            raise ValueError(f"kv_norm_rope: head_dim {d}, qkv width {qkv.shape[1]}")
        dst = meta["unified"]["row_dst"]
        if dst.shape[0] != n:
            raise ValueError(f"row_dst has {dst.shape[0]} rows, qkv {n}")
        layer = meta["layer"]
        k_pool, v_pool = self.arena.layer_kv(layer)
        self._check_pools(k_pool, v_pool)
        cache = self._rope_cache()
        _lib.call("qx_qk_norm_rope_kv", _ptr(qkv), qkv.stride(0), None, 0,
                  _ptr(k_pool), _ptr(v_pool), _ptr(dst), None, None, None, _ptr(cache),
                  int(cache.dtype == torch.float32), _ptr(positions), _ptr(attn.q_norm.weight),
                  _ptr(attn.k_norm.weight), n, hq, hk, d, float(attn.q_norm.variance_epsilon),
                  int(v_pool.dtype == torch.float16), _stream())
        meta["kv_fresh_layer"] = layer
        meta["q_norm_on_load"] = (positions, attn)
        return qkv[:, :hq * d]

    @staticmethod
    def _check_pools(k_pool, v_pool):
        """K pools are bf16; V pools bf16 (the reference KVArena's,
        arena.py:111-121) or fp16 (an arena of this engine's own that keeps
        V in fp16: the PV product then runs with fp16 probabilities)."""
        if k_pool.dtype != torch.bfloat16:
            raise ValueError(f"K pool dtype {k_pool.dtype}: K pages are bf16")
        if v_pool.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError(f"V pool dtype {v_pool.dtype}: V pages are bf16 or fp16")

    def _v_dtype(self):
        return self.arena.layer_kv(0)[1].dtype

    def kv_row_scatter(self, k3, v3, src, dst, layer):
        """Scatter KV rows into the layer's arena pages; dst < 0 is padding.
        bf16 V rows going to an fp16 V pool are converted (saturated at
        +-65504); rows already of the pool's type (the tail copy) are copied."""
        count = src.shape[0]
        row = self.num_kv_heads * self.head_dim
        k_pool, v_pool = self.arena.layer_kv(layer)
        self._check_pools(k_pool, v_pool)
        if k3.dtype != torch.bfloat16:
            raise ValueError(f"K rows dtype {k3.dtype}: K pages are bf16")
        if v3.dtype == v_pool.dtype:
            convert = 0
        elif v3.dtype == torch.bfloat16 and v_pool.dtype == torch.float16:
            convert = 1
        else:
            raise ValueError(f"V rows of {v3.dtype} cannot go to a {v_pool.dtype} pool")
        _lib.call("qx_kv_scatter", _ptr(k3), k3.stride(0), _ptr(v3), v3.stride(0), _ptr(k_pool),
                  _ptr(v_pool), _ptr(src), _ptr(dst), count, row, convert, _stream())

    def write_kv(self, k3, v3, meta, *, copy_tail=True):
        """Write fresh rows and retained partial pages (attention.py:1175-1195)."""
        if meta.get("kv_written", False):
            return
        layer = meta["layer"]
        pool = meta["unified"]
        if pool is None:
            return
        # qk_norm_rope_kv already wrote this layer's fresh rows
        fresh = meta.pop("kv_fresh_layer", None) != layer
        if fresh and pool["src"].numel():
            if k3 is None:
                raise ValueError(f"layer {layer}: no K/V rows and none written by "
                                 "qk_norm_rope_kv")
            self.kv_row_scatter(k3, v3, pool["src"], pool["dst"], layer)
        if copy_tail and pool.get("tail_src") is not None:
            k_pool, v_pool = self.arena.layer_kv(layer)
            self.kv_row_scatter(k_pool, v_pool, pool["tail_src"], pool["tail_dst"], layer)

    def attention(self, q, k, v, chunk, *, output=None):
        """Attention over the chunk and the arena; the quantized o_proj input.

        q, k and v are the flat per-row projections; v may be the strided
        slice of qkv. Returns (e4m3 rows, col-major scales).
        """
        n = q.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        if chunk.attention_mode not in ("unified", "tree"):
            raise ValueError(f"attention mode {chunk.attention_mode!r}")
        for key in ("shared", "canvas"):
            if chunk.meta.get(key) is not None:
                raise ValueError(f"this engine has no {key}-row attention path")
        q3 = q.view(n, hq, d)
        k3, v3 = self._kv_views(n, k, v)
        if chunk.attention_mode == "tree":
            if k3 is None:
                raise ValueError("the tree path reads the pack's own K and V rows")
            return self.attention_tree(q3, k3, v3, chunk.meta, output=output)
        return self.attention_unified(q3, k3, v3, chunk.meta, output=output)

    def _kv_views(self, n, k, v):
        """(n, HK, D) views of flat K and V rows; None when qk_norm_rope_kv
        wrote them to the pages already."""
        if k is None:
            return None, None
        hk, d = self.num_kv_heads, self.head_dim
        return k.view(n, hk, d), v.view(n, hk, d) if v.is_contiguous() else v

    def attention_tree(self, q3, k3, v3, meta, *, output=None, quantize=True):
        """The tree attention path (attention.py:1395-1441): the pack's KV
        writes into arena pages, then call A (causal over the pack's own rows
        in `cu_a` segments), call B (the reader rows over resident pages, not
        causal; label-path rows also over their ancestor rows, call C, merged
        into B), each with its log-sum-exp, and one fused merge + o_proj
        input quantization (attention.py:902-948). Returns (e4m3, scales),
        or with quantize=False the merged bf16 rows (for tests)."""
        n = q3.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        layer = meta["layer"]
        dev = q3.device
        written = meta.pop("kv_fresh_layer", None) == layer   # by qk_norm_rope_rows
        if meta.get("kv_src") is not None and meta["kv_src"].numel() and not written:
            self.kv_row_scatter(k3, v3, meta["kv_src"], meta["kv_dst"], layer)
        # call A reads the pack's own K and V rows contiguous (as
        # qk_norm_rope_rows gives them, else one identity scatter)
        row = hk * d
        v_dtype = self._v_dtype()
        if k3.is_contiguous() and v3.is_contiguous() and v3.dtype == v_dtype:
            k_rows, v_rows = k3.reshape(n, row), v3.reshape(n, row)
        else:
            k_rows = torch.empty((n, row), dtype=torch.bfloat16, device=dev)
            v_rows = torch.empty((n, row), dtype=v_dtype, device=dev)
            _lib.call("qx_kv_scatter", _ptr(k3), k3.stride(0), _ptr(v3), v3.stride(0),
                      _ptr(k_rows), _ptr(v_rows), None, None, n, row,
                      int(v3.dtype != v_dtype), _stream())
        scale = float(d ** -0.5)
        seg = meta["segments"]
        out_a = torch.empty((n, hq * d), dtype=torch.bfloat16, device=dev)
        lse_a = torch.empty((hq, max(n, 1)), dtype=torch.float32, device=dev)
        self._lse_call(q3, None, k_rows, v_rows, seg, None, seg["cu_q"], scale, out_a, lse_a)
        reads = meta["reads"]
        if output is not None:
            o_q, o_s = output
        else:
            o_q = torch.empty((n, hq * d), dtype=self.fp8, device=dev)
            o_s = self._col_major_scales(n, hq * d, dev)
        if reads is None:
            meta["layer"] += 1
            return self.quant(out_a, output=(o_q, o_s)) if quantize else out_a
        nb = reads["rows"].shape[0]
        k_pool, v_pool = self.arena.layer_kv(layer)
        out_b = torch.empty((nb, hq * d), dtype=torch.bfloat16, device=dev)
        lse_b = torch.empty((hq, max(nb, 1)), dtype=torch.float32, device=dev)
        self._lse_call(q3, reads["rows"], k_pool, v_pool, reads, reads["table"], None, scale,
                       out_b, lse_b)
        if reads.get("nodes") is not None:
            self._call_c(q3, k_rows, v_rows, reads["nodes"], scale, out_b, lse_b)
        args = (_ptr(out_a), out_a.stride(0), _ptr(out_b), out_b.stride(0), _ptr(lse_a),
                lse_a.stride(0), _ptr(lse_b), lse_b.stride(0), _ptr(reads["source"]), n, hq, d)
        if d == GROUP and quantize:
            _lib.call("qx_merge_attn_quant", *args, _ptr(o_q), o_q.stride(0), _ptr(o_s),
                      self._scale_ld(o_s), _stream())
        else:
            # a 128-column FP8 group spans several heads: bf16 merge, then quant
            merged = torch.empty((n, hq * d), dtype=torch.bfloat16, device=dev)
            _lib.call("qx_merge_attn_quant", *args, _ptr(merged), merged.stride(0), None, 0,
                      _stream())
            if not quantize:
                meta["layer"] += 1
                return merged
            self.quant(merged, output=(o_q, o_s))
        meta["layer"] += 1
        return o_q, o_s

    def _call_c(self, q3, k_rows, v_rows, nodes, scale, out_b, lse_b):
        """Call C (attention.py:1424-1434): label-path rows over the rows
        above their first node (gathered from the pack's own K and V rows),
        not causal, merged into their call B rows (merge_partial)."""
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        dev = q3.device
        nq = nodes["rows"].shape[0]
        nk = nodes["key_rows"].shape[0]
        row = hk * d
        k_c = torch.empty((nk, row), dtype=torch.bfloat16, device=dev)
        v_c = torch.empty((nk, row), dtype=v_rows.dtype, device=dev)
        into = nodes.get("gather_rows")
        if not torch.is_tensor(into):
            into = torch.arange(nk, dtype=torch.int64, device=dev)
        _lib.call("qx_kv_scatter", _ptr(k_rows), k_rows.stride(0), _ptr(v_rows), v_rows.stride(0),
                  _ptr(k_c), _ptr(v_c), _ptr(nodes["key_rows"]), _ptr(into), nk, row, 0,
                  _stream())
        out_c = torch.empty((nq, hq * d), dtype=torch.bfloat16, device=dev)
        lse_c = torch.empty((hq, max(nq, 1)), dtype=torch.float32, device=dev)
        self._lse_call(q3, nodes["rows"], k_c, v_c, nodes, None, nodes["cu_k"], scale, out_c,
                       lse_c)
        _lib.call("qx_merge_partial", _ptr(out_b), out_b.stride(0), _ptr(lse_b), lse_b.stride(0),
                  _ptr(nodes["b_index"]), _ptr(out_c), out_c.stride(0), _ptr(lse_c),
                  lse_c.stride(0), nq, hq, d, _stream())

    def _lse_call(self, q3, q_index, k, v, tables, table, cu_k, scale, out, lse):
        """One qx_attention_lse call over `tables` (cu_q, used, max_q,
        max_used, causal, work): paged through `table`, or over contiguous
        rows at `cu_k`."""
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        work = tables.get("work")
        if not torch.is_tensor(work):
            work = None
        n_work = int(tables.get("n_work", 0)) if work is not None else 0
        seqs = tables["used"].shape[0]
        _lib.call("qx_attention_lse", _ptr(q3), q3.stride(0), _ptr(q_index), _ptr(k), _ptr(v),
                  _ptr(tables["cu_q"]), _ptr(tables["used"]), _ptr(table),
                  table.stride(0) if table is not None else 0, _ptr(cu_k), seqs,
                  int(tables["max_q"]), int(tables["max_used"]), hq, hk, d, scale,
                  int(tables.get("causal", True)), _ptr(out), out.stride(0), _ptr(lse),
                  lse.stride(0), _ptr(work), n_work, int(v.dtype == torch.bfloat16), _stream())

    def attention_unified(self, q3, k3, v3, meta, *, softmax_scale=None, output=None):
        """Write the chunk's KV to its pages, then one paged causal call with
        the o_proj input quantization fused (attention.py:1477-1573)."""
        if meta["unified"] is None:
            raise ValueError("this engine reads KV from arena pages; pack with pages")
        self.write_kv(k3, v3, meta)
        out = self._paged(q3, meta["unified"], meta["layer"], softmax_scale, output,
                          qnorm=meta.pop("q_norm_on_load", None))
        meta["layer"] += 1
        return out

    def write_kv_only(self, q, k, v, chunk):
        """A layer whose attention output no row reads (the last layer of a
        pass of prefill pieces): only its K and V rows go to the pages."""
        n = q.shape[0]
        k3, v3 = self._kv_views(n, k, v)
        meta = chunk.meta
        if chunk.attention_mode == "tree":
            layer = meta["layer"]
            written = meta.pop("kv_fresh_layer", None) == layer
            if meta.get("kv_src") is not None and meta["kv_src"].numel() and not written:
                self.kv_row_scatter(k3, v3, meta["kv_src"], meta["kv_dst"], layer)
        else:
            self.write_kv(k3, v3, meta)
        meta.pop("q_norm_on_load", None)
        meta["layer"] += 1

    def attention_final(self, q, k, v, chunk, rows):
        """The last layer's attention: write the pack's KV (every row: later
        packs may borrow it), then attend only for `rows` (the pass's final
        rows) through meta["final_query"], one query per row seeing exactly
        the keys it sees inside its own sequence. Returns the o_proj input of
        those rows, bit-identical to theirs in the full call."""
        n = q.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        meta = chunk.meta
        fq = meta.get("final_query")
        if fq is None or meta["unified"] is None:
            raise ValueError("the pack carries no final-row attention metadata")
        k3, v3 = self._kv_views(n, k, v)
        self.write_kv(k3, v3, meta)
        qf = q.view(n, hq, d).index_select(0, rows)
        qnorm = meta.pop("q_norm_on_load", None)
        if qnorm is not None:
            qnorm = (qnorm[0].index_select(0, rows), qnorm[1])
        out = self._paged(qf, fq, meta["layer"], None, None, qnorm=qnorm)
        meta["layer"] += 1
        return out

    def _paged(self, q3, tables, layer, softmax_scale, output, qnorm=None):
        """One paged causal call over `tables` (cu_q, used, table, max_q,
        max_used) with the o_proj input quantization fused. qnorm =
        (positions of q3's rows, attention module): q3 is the raw q of the
        qkv projection, normalized and rotated as the kernel loads it."""
        n = q3.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        k_pool, v_pool = self.arena.layer_kv(layer)
        self._check_pools(k_pool, v_pool)
        v_bf16 = int(v_pool.dtype == torch.bfloat16)
        scale = d ** -0.5 if softmax_scale is None else softmax_scale
        table = tables["table"]
        if output is not None:
            o_q, o_s = output
        else:
            o_q = torch.empty((n, hq * d), dtype=self.fp8, device=q3.device)
            o_s = self._col_major_scales(n, hq * d, q3.device)
        seqs = tables["used"].shape[0]
        q_ld = q3.stride(0)
        args = (_ptr(k_pool), _ptr(v_pool), _ptr(tables["cu_q"]), _ptr(tables["used"]),
                _ptr(table), table.stride(0), seqs, int(tables["max_q"]),
                int(tables["max_used"]), hq, hk, d, self.arena.page_tokens, float(scale),
                int(tables.get("causal", True)))
        # the pack's work list (one item per real query tile), when it has
        # one, and the query rows per item it was built for
        work = tables.get("work")
        if not torch.is_tensor(work):
            work = None
        n_work = int(tables.get("n_work", 0)) if work is not None else 0
        rows = int(tables.get("work_rows", 0)) if work is not None else 0
        if qnorm is not None:
            positions, attn = qnorm
            if d != GROUP or positions.shape[0] != n:
                raise ValueError("q-norm on load: head_dim 128 and one position per row")
            cache = self._rope_cache()
            _lib.call("qx_paged_attention_qnorm", _ptr(q3), q_ld, *args, _ptr(o_q),
                      o_q.stride(0), _ptr(o_s), self._scale_ld(o_s), _ptr(work), n_work, rows,
                      v_bf16, _ptr(positions), _ptr(cache), int(cache.dtype == torch.float32),
                      _ptr(attn.q_norm.weight), float(attn.q_norm.variance_epsilon), _stream())
        elif d == GROUP:
            _lib.call("qx_paged_attention", _ptr(q3), q_ld, *args, None, _ptr(o_q),
                      o_q.stride(0), _ptr(o_s), self._scale_ld(o_s), _ptr(work), n_work, rows,
                      v_bf16, _stream())
        else:
            # a 128-column FP8 group spans several heads: bf16 out, then quant
            o = torch.empty((n, hq * d), dtype=torch.bfloat16, device=q3.device)
            _lib.call("qx_paged_attention", _ptr(q3), q_ld, *args, _ptr(o), None, o.stride(0),
                      None, 0, _ptr(work), n_work, rows, v_bf16, _stream())
            self.quant(o, output=(o_q, o_s))
        return o_q, o_s

    def attention_bf16(self, q3, meta, layer):
        """The unquantized attention rows of one layer (for tests)."""
        n = q3.shape[0]
        hq, hk, d = self.num_q_heads, self.num_kv_heads, self.head_dim
        unified = meta["unified"]
        k_pool, v_pool = self.arena.layer_kv(layer)
        o = torch.empty((n, hq * d), dtype=torch.bfloat16, device=q3.device)
        table = unified["table"]
        _lib.call("qx_paged_attention", _ptr(q3), q3.stride(0), _ptr(k_pool), _ptr(v_pool),
                  _ptr(unified["cu_q"]), _ptr(unified["used"]), _ptr(table), table.stride(0),
                  unified["used"].shape[0], int(unified["max_q"]), int(unified["max_used"]),
                  hq, hk, d,
                  self.arena.page_tokens, float(d ** -0.5), int(unified.get("causal", True)),
                  _ptr(o), None, o.stride(0), None, 0, None, 0, 0,
                  int(v_pool.dtype == torch.bfloat16), _stream())
        return o
