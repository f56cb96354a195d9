"""PreparedAttention: the shared-KV INT8 attention operator on MI355X.

Interface counterpart: npu_sparse_attn_sharedkv_int8/attention.py:19-257 of the
reference checkout.  The constructor signature, the validation (ValueError on
contract violations, RuntimeError on ABI drift), the retained attributes
(.case, .out, .lse, .args, .workspace, .partial, .blocks, .splits, .variant,
.c8_dynamic) and _rebind_same_geometry() are kept, so serving code written
for the reference runs unchanged with device tensors on "cuda" (HIP).

Everything is validated and every buffer is allocated here, outside graph
capture; run() only launches the HIP kernel on the caller's current stream.
The only kernel family in this build is the C8 one (c8_attention.py).  It
also serves what the reference routes to its legacy Ascend variants for
window-only (ratio 1) launches, explicit original slots (draft/MTP
ori_indices) and head counts other than eight (groups of eight heads per
work-group; above eight heads the Q/P residuals are off, as in the
reference's model).
"""
import torch

from . import c8_attention
from .runtime import SharedKVArgs

_Args = SharedKVArgs


def _check_cache(cache, table, scale, batch, device):
    """Same conditions as the reference's check_cache (attention.py:42-53)."""
    if cache is None or cache.dtype != torch.int8 or cache.ndim != 4 or tuple(cache.shape[-2:]) != (1, 512):
        raise ValueError("Expected INT8 cache[P,B,1,512]")
    pages, block = cache.shape[0], cache.shape[1]
    if (pages == 0 or block == 0 or pages * block >= 2 ** 31 or cache.stride(1) != 512
            or cache.stride(-1) != 1 or cache.stride(0) < block * 512):
        raise ValueError("Invalid page stride or empty cache")
    if (table is None or table.ndim != 2 or table.shape[0] != batch or table.dtype != torch.int32
            or not table.is_contiguous()):
        raise ValueError("Expected contiguous INT32 block table[B,num_pages]")
    if scale is None or tuple(scale.shape) != (512,) or scale.dtype != torch.float32 or not scale.is_contiguous():
        raise ValueError("Expected frozen contiguous FP32 scale[512]")
    if any(x.device != device for x in (cache, table, scale)):
        raise ValueError("All inputs must be on the same GPU")


class PreparedAttention:
    """Retains all input, output and scratch storage; run() allocates nothing
    and reads nothing back from the device.

    Protocol: BF16 Q[T,8,512]; INT8 caches [P,32,1,512] with any page stride
    that is a multiple of 16 bytes; frozen FP32[512] scales per cache kind;
    ratio 4 (window + top-k compressed rows, top-k <= 1024) or 128 (window +
    every compressed row); window 128.
    """

    def __init__(self, case, ori_scale, cmp_scale=None, *, output=None, splits=None, tile_size=None,
                 query_group=None, max_seq_len=None, return_lse=False, lse_output=None,
                 scratch_allocator=None, adaptive_splits=False, trim_cube_tails=None, dynamic_c4=None,
                 dynamic_c128=None, dynamic_grouped_c128=None, implementation="auto"):
        if implementation not in ("auto", "v65", "fallback"):
            raise ValueError("implementation must be auto, v65 or fallback")
        q = case.q
        if q.device.type != "cuda" or q.dtype != torch.bfloat16 or q.ndim != 3 or q.shape[-1] != 512:
            raise ValueError("Expected BF16 Q[T,H,512] on a GPU")
        tokens, heads, _ = q.shape
        if not heads or heads > 128 or not q.is_contiguous():
            raise ValueError("Expected 1..128 heads and contiguous Q")
        if case.ratio not in (1, 4, 128) or case.window <= 0:
            raise ValueError("Expected SWA/C4/C128 and a positive window")
        device = q.device
        batch = case.seq_lens.numel()
        _check_cache(case.ori, case.ori_block_table, ori_scale, batch, device)
        if case.ratio != 1:
            _check_cache(case.cmp, case.cmp_block_table, cmp_scale, batch, device)
        if case.ratio == 4:
            ix = case.cmp_indices
            if (ix is None or ix.ndim != 3 or tuple(ix.shape[:2]) != (tokens, 1) or ix.shape[2] == 0
                    or ix.dtype != torch.int32 or not ix.is_contiguous()):
                raise ValueError("C4 requires contiguous INT32 indices[T,1,topk]")
        if (tuple(case.cu_q.shape) != (batch + 1,) or case.seq_lens.ndim != 1
                or tuple(case.sink.shape) != (heads,)):
            raise ValueError("Invalid sequence metadata or sink shape")
        for x, dtype in ((case.cu_q, torch.int32), (case.seq_lens, torch.int32), (case.sink, torch.float32)):
            if x.dtype != dtype or x.device != device or not x.is_contiguous():
                raise ValueError("Invalid metadata dtype, device or contiguity")
        if case.cmp_indices is not None and case.cmp_indices.device != device:
            raise ValueError("Indices must be on the same GPU")
        if case.ori_indices is not None:
            ix = case.ori_indices
            if (ix.ndim != 3 or tuple(ix.shape[:2]) != (tokens, 1) or ix.shape[-1] == 0
                    or ix.dtype != torch.int32 or ix.device != device or not ix.is_contiguous()):
                raise ValueError("Original physical slots must be contiguous INT32[T,1,K] on the query device")

        self.case = case
        self.scales = ori_scale, cmp_scale
        self.out = output if output is not None else torch.empty_like(q)
        if (tuple(self.out.shape) != tuple(q.shape) or self.out.device != device
                or self.out.dtype != torch.bfloat16 or not self.out.is_contiguous()):
            raise ValueError("Invalid output buffer")
        if lse_output is not None:
            self.lse = lse_output
        else:
            self.lse = torch.empty((tokens, heads), dtype=torch.float32, device=device) if return_lse else None
        if self.lse is not None and (tuple(self.lse.shape) != (tokens, heads) or self.lse.dtype != torch.float32
                                     or self.lse.device != device or not self.lse.is_contiguous()):
            raise ValueError("Invalid FP32 LSE[T,H] output buffer")

        # Tuning knobs of the Ascend planner.  Only the ones that change this
        # build's numerics (tile_size, splits, query_group) are honoured; the
        # rest are validated for type and recorded.  adaptive_splits has
        # nothing left to switch: the kernel always adapts the partition count
        # to the live rows of a padded launch (c8_attention.device_splits).
        # query_group 2 or 4 on a launch of at most eight heads without
        # explicit slots runs the grouped plan (reference.py:224-323 with
        # that query_group).  As in the reference's operator
        # (attention.py:104-112 there) its tiles are 256 keys and it runs one
        # KV partition unless told otherwise (launch_sharedkv_c8_dense_paired
        # / _packed); tile_size=128 runs it on 128-key tiles at the library's
        # partition plan (..._paired_narrow / _packed_narrow), and explicit
        # splits apply to either.  C4 groups take the dense multiplicity list
        # of reference.py:246-249 at any sequence length (the reference's
        # operator accepts grouped C4 only under max_seq_len <= 1024,
        # attention.py:88-98 there).  Any other request runs the ungrouped
        # plan on 128-key tiles, and self.query_group / self.tile_size tell
        # callers which plan ran (the reference's C8 path likewise runs its
        # kernel's own plan, c8_attention.py:74-113; its tests rebuild the
        # oracle plan from the device's choice, attention_cases.py:56-111).
        if query_group not in (None, 1, 2, 4):
            raise ValueError("query_group must be 1, 2 or 4")
        if splits is not None and (not isinstance(splits, int) or not 1 <= splits <= c8_attention.MAX_SPLITS):
            raise ValueError(f"Expected 1..{c8_attention.MAX_SPLITS} KV partitions")
        paired = query_group in (2, 4) and heads <= c8_attention.HEADS and case.ori_indices is None
        allowed = (c8_attention.TILE, c8_attention.GROUPED_TILE) if paired else (c8_attention.TILE,)
        if tile_size is not None and tile_size not in allowed:
            raise ValueError(f"tile_size must be None or one of {allowed} for this plan (grouped plans: 128 or 256 "
                             f"keys, others: 128)")
        self.tile_size = (tile_size or c8_attention.GROUPED_TILE) if paired else c8_attention.TILE
        self.query_group = query_group if paired else 1
        self.adaptive_splits = bool(adaptive_splits)
        self.trim_cube_tails = bool(trim_cube_tails)
        self.dynamic_c4 = self.dynamic_c128 = self.dynamic_grouped_c128 = False
        self.max_seq_len = max_seq_len
        self.device_index = device.index if device.index is not None else torch.cuda.current_device()
        self.c8_dynamic = False
        self.workspace = self.partial = None

        if tokens == 0:
            self.blocks, self.splits, self.variant = 0, 1, None
            self.args = None
            return
        ori_topk = case.ori_indices.shape[-1] if case.ori_indices is not None else 0
        if splits is not None:
            self.splits = splits
        elif paired:
            self.splits = (1 if self.tile_size == c8_attention.GROUPED_TILE
                           else c8_attention.choose_paired_splits(tokens, case.ratio, max_seq_len))
        else:
            self.splits = c8_attention.choose_splits(
                tokens * c8_attention.head_groups(heads), case.ratio,
                case.cmp_indices.shape[-1] if case.ratio == 4 else 0, max_seq_len, ori_topk)

        ptr = lambda t: t.data_ptr() if t is not None else 0  # noqa: E731
        cmp = case.cmp if case.ratio != 1 else None
        self.args = _Args(
            q=ptr(q), ori=ptr(case.ori), cmp=ptr(cmp), oriScale=ptr(ori_scale),
            cmpScale=ptr(cmp_scale if case.ratio != 1 else None), oriTable=ptr(case.ori_block_table),
            cmpTable=ptr(case.cmp_block_table if case.ratio != 1 else None),
            indices=ptr(case.cmp_indices if case.ratio == 4 else None), cuQ=ptr(case.cu_q),
            seqLens=ptr(case.seq_lens), sinks=ptr(case.sink), out=ptr(self.out), workspace=0, lse=ptr(self.lse),
            oriStride=case.ori.stride(0), cmpStride=cmp.stride(0) if cmp is not None else 0, partial=0,
            oriIndices=ptr(case.ori_indices), tokens=tokens, heads=heads, batch=batch,
            oriBlock=case.ori.shape[1], cmpBlock=cmp.shape[1] if cmp is not None else 0,
            oriTableWidth=case.ori_block_table.shape[1],
            cmpTableWidth=case.cmp_block_table.shape[1] if cmp is not None else 0, ratio=case.ratio,
            window=case.window, topk=case.cmp_indices.shape[-1] if case.ratio == 4 else 0, splits=self.splits,
            oriTopk=case.ori_indices.shape[-1] if case.ori_indices is not None else 0, oriPages=case.ori.shape[0],
            softmaxScale=case.softmax_scale)
        self.blocks = tokens * c8_attention.head_groups(heads) * self.splits

        if implementation == "fallback" or (implementation == "auto" and not c8_attention.enabled()):
            raise ValueError("The legacy (non-C8) kernels are not part of the MI355X build; "
                             "use implementation='auto' with SHAREDKV_C8_DECODE=1")
        if not c8_attention.supported(self):
            raise ValueError("This ABI is outside the C8 path (needs ratio 1/4/128, window 128, "
                             "block32 pages, top-k <= 1024, at most 1024 explicit original slots)")
        prepared = c8_attention.prepare(self, scratch_allocator=scratch_allocator)
        self.__dict__.update(prepared.__dict__)
        if paired:
            wide = self.tile_size == c8_attention.GROUPED_TILE
            self.variant = ((c8_attention.VARIANT_DENSE_PAIRED if wide else c8_attention.VARIANT_PAIRED_NARROW)
                            if query_group == 2 else
                            (c8_attention.VARIANT_DENSE_PACKED if wide else c8_attention.VARIANT_PACKED_NARROW))

    def _rebind_same_geometry(self, case, *, output=None, lse_output=None):
        """Serving fast path: same geometry, new tensors (attention.py:233-247)."""
        self.case = case
        if output is not None:
            self.out, self.lse = output, lse_output
        if not self.blocks:
            return
        if output is not None:
            self.args.out = output.data_ptr()
            self.args.lse = lse_output.data_ptr() if lse_output is not None else 0
        for name, tensor in (("q", case.q), ("ori", case.ori), ("cmp", case.cmp if case.ratio != 1 else None),
                             ("oriTable", case.ori_block_table),
                             ("cmpTable", case.cmp_block_table if case.ratio != 1 else None),
                             ("indices", case.cmp_indices if case.ratio == 4 else None), ("cuQ", case.cu_q),
                             ("seqLens", case.seq_lens), ("sinks", case.sink), ("oriIndices", case.ori_indices)):
            setattr(self.args, name, tensor.data_ptr() if tensor is not None else 0)

    def device_splits(self, cu_q=None, seq_lens=None, merge_mode=0):
        """KV partitions the kernel uses for this launch under live metadata
        (default: the case's, read back to the host); equals .splits unless
        graph padding leaves rows idle.  merge_mode is the library's
        (sharedkv_c8_set_merge_mode): 1 keeps the launch plan."""
        if not self.blocks or self.query_group != 1:
            return self.splits          # the paired plan keeps the launch's partitions
        c = self.case
        cu_q = c.cu_q.cpu().tolist() if cu_q is None else cu_q
        seq_lens = c.seq_lens.cpu().tolist() if seq_lens is None else seq_lens
        return c8_attention.device_splits(self.splits, self.args.tokens, self.args.heads, self.args.ratio,
                                          self.args.topk, cu_q, seq_lens, self.args.oriTopk,
                                          fused=merge_mode == 0,
                                          cmp_rows=self.args.cmpTableWidth * c8_attention.BLOCK)

    def run(self):
        """Launch on the current stream of the case's device; returns .out."""
        if self.blocks == 0:
            return self.out
        self.native.attention(self.argument_address, self.blocks, self.variant, self.device_index)
        return self.out
