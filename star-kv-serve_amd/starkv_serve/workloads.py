"""Seeded synthetic decode workloads in the reference's cache layout.

Used by the benchmark, the smoke check and the tests; nothing here runs in the
decode path itself. Inputs follow the reference benchmark configurations:

* K ranks per head drawn from {16, 32, 48, 64} (widths = ranks rounded to 16,
  offsets = prefix sums, checkpoint.py:125-128), one head-shared V rank per layer;
* physical pages: block 0 is the null block, pages 1..N are a random permutation,
  filled into each request's block-table row in order; block size 16 unless given;
* codes, queries ~ N(0, 1); K bases N(0, 1) / sqrt(rank), V bases N(0, 1) / sqrt(r_v);
  scale 1/sqrt(128); cos_sin_cache[p] = [cos(p theta) | sin(p theta)],
  theta_i = 10000^(-2i/128), computed in fp32 and stored in the model dtype;
* 3.2-bit layers: codes rotated per head by the block Hadamard (seed 1234, one
  generator per projection, heads in order, checkpoint.py:96-103) with the bases
  counter-rotated, then packed with ``pack_kv``.

Tensors are drawn from one CPU ``torch.Generator`` per workload (or on the GPU
for benchmark-sized caches), so every consumer sees identical bytes.
"""
import math
from dataclasses import dataclass, field

import torch

HEAD_DIM = 128
BLOCK_SIZE = 16
RANK_CHOICES = (16, 32, 48, 64)


def align16(n: int) -> int:
    return (int(n) + 15) // 16 * 16


def cos_sin_table(max_pos: int, dtype, device="cpu", base: float = 10000.0) -> torch.Tensor:
    inv_freq = 1.0 / (base ** (torch.arange(0, HEAD_DIM, 2, dtype=torch.float32) / HEAD_DIM))
    t = torch.arange(max_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    return torch.cat([freqs.cos(), freqs.sin()], dim=-1).to(dtype).to(device)


@dataclass
class Workload:
    """One decode call's operands, named as the reference kernels name them."""
    query: torch.Tensor
    kv_cache: torch.Tensor
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    max_seq_len: int
    k_up: torch.Tensor
    k_ranks: torch.Tensor
    k_head_offsets: torch.Tensor
    k_width: int
    v_up_by_q: torch.Tensor
    cos_sin_cache: torch.Tensor
    scale: float
    ranks: list
    v_rank: int
    lengths: list
    quant: bool = False
    row: object = None
    k_nouts: torch.Tensor = None
    head_of_lane: torch.Tensor = None
    k_tiles: tuple = None
    k_codes: torch.Tensor = None      # per-token codes in token order (b, l), for the write path
    v_codes: torch.Tensor = None
    extra: dict = field(default_factory=dict)

    @property
    def n(self) -> int:
        return self.query.shape[0]

    @property
    def tokens(self) -> int:
        return int(sum(self.lengths))

    def to(self, device) -> "Workload":
        out = {}
        for k, v in self.__dict__.items():
            if isinstance(v, torch.Tensor):
                out[k] = v.to(device)
            elif isinstance(v, tuple) and v and isinstance(v[0], torch.Tensor):
                out[k] = tuple(x.to(device) for x in v)
            else:
                out[k] = v
        return Workload(**out)

    def decode_args(self) -> tuple:
        if self.quant:
            return (self.query, self.kv_cache, self.block_table, self.seq_lens, self.max_seq_len, self.row,
                    self.k_up, self.head_of_lane, self.k_tiles, self.v_up_by_q, self.cos_sin_cache, self.scale)
        return (self.query, self.kv_cache, self.block_table, self.seq_lens, self.max_seq_len, self.k_up,
                self.k_ranks, self.k_head_offsets, self.k_width, self.v_up_by_q, self.cos_sin_cache, self.scale)

    def bytes_per_step(self) -> int:
        """Algorithmic HBM bytes of one decode call: every valid cache row once, the
        block-table entries, q and out, the bases and the cos/sin rows."""
        row = self.row.nbytes if self.quant else (self.k_width + self.v_rank) * self.kv_cache.element_size()
        bs = self.kv_cache.shape[1]
        pages = sum((L + bs - 1) // bs for L in self.lengths)
        n, H = self.query.shape[0], self.query.shape[1]
        es = self.query.element_size()
        return (self.tokens * row + pages * 4 + 2 * n * H * HEAD_DIM * es + self.k_up.numel() * self.k_up.element_size()
                + self.v_up_by_q.numel() * self.v_up_by_q.element_size()
                + max(self.lengths) * HEAD_DIM * self.cos_sin_cache.element_size())

    def flops_per_step(self) -> int:
        """2*128*W per token for the K logits, 2*H*r_v per token for P @ V, plus the lift."""
        n, H = self.query.shape[0], self.query.shape[1]
        W = (H // len(self.ranks)) * self.k_width
        return self.tokens * (2 * HEAD_DIM * W + 2 * H * self.v_rank) + n * 2 * H * self.v_rank * HEAD_DIM


def _page_layout(lengths, gen, extra_blocks=0, block_size=BLOCK_SIZE):
    pages = [(L + block_size - 1) // block_size for L in lengths]
    total = sum(pages)
    perm = (torch.randperm(total, generator=gen) + 1).to(torch.int32) if total else torch.zeros(0, dtype=torch.int32)
    max_blocks = max(1, max(pages) if pages else 1)
    bt = torch.zeros(len(lengths), max_blocks, dtype=torch.int32)
    o = 0
    for b, p in enumerate(pages):
        bt[b, :p] = perm[o:o + p]
        o += p
    return bt, total + 1 + extra_blocks


def _token_slots(lengths, bt, block_size=BLOCK_SIZE):
    """(block, slot) for every token in (b, l) order."""
    blocks, slots = [], []
    for b, L in enumerate(lengths):
        l = torch.arange(L)
        blocks.append(bt[b, (l // block_size)].long())
        slots.append(l % block_size)
    if not blocks:
        return torch.zeros(0, dtype=torch.long), torch.zeros(0, dtype=torch.long)
    return torch.cat(blocks), torch.cat(slots)


def make_lowrank(lengths, num_heads=32, num_kv_heads=None, ranks=None, v_rank=64, seed=0, dtype=torch.bfloat16,
                 max_seq_len=None, col_pad=0, poison=True, peaked=1.0, gen_device="cpu",
                 rank_choices=RANK_CHOICES, block_size=BLOCK_SIZE) -> Workload:
    """bf16/fp16 low-rank workload. `col_pad` > 0 makes the cache a column slice of a
    wider buffer (strided view); `poison` fills unused slots with NaN."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    Hkv = num_kv_heads or num_heads
    if ranks is None:
        ranks = [rank_choices[i] for i in torch.randint(0, len(rank_choices), (Hkv,), generator=gen).tolist()]
    widths = [align16(r) for r in ranks]
    offsets = [sum(widths[:h]) for h in range(Hkv)]
    W = sum(widths)
    n = len(lengths)
    max_seq_len = max_seq_len or max(max(lengths), 1)
    bt, nblocks = _page_layout(lengths, gen, block_size=block_size)
    width = W + v_rank

    q = (torch.randn(n, num_heads, HEAD_DIM, generator=gen) * peaked).to(dtype)
    k_up = torch.zeros(W, HEAD_DIM)
    for h in range(Hkv):
        k_up[offsets[h]:offsets[h] + ranks[h]] = torch.randn(ranks[h], HEAD_DIM, generator=gen) / math.sqrt(ranks[h])
    k_up = k_up.to(dtype)
    v_up_by_q = (torch.randn(num_heads, v_rank, HEAD_DIM, generator=gen) / math.sqrt(v_rank)).to(dtype)
    cs = cos_sin_table(max(max_seq_len, max(lengths) + 1), dtype)

    T = int(sum(lengths))
    blk, slot = _token_slots(lengths, bt, block_size)
    if gen_device == "cpu":
        k_codes = torch.randn(T, W, generator=gen).to(dtype)
        v_codes = torch.randn(T, v_rank, generator=gen).to(dtype)
        for h in range(Hkv):  # lanes between a head's rank and its width hold zero codes
            k_codes[:, offsets[h] + ranks[h]:offsets[h] + widths[h]] = 0
        buf = torch.full((nblocks, block_size, width + col_pad), float("nan") if poison else 0.0, dtype=dtype)
        buf[0] = 0  # the null block holds finite codes
        cache = buf[:, :, :width]
        cache[blk, slot, :W] = k_codes
        cache[blk, slot, W:] = v_codes
    else:
        g2 = torch.Generator(device=gen_device).manual_seed(seed + 7919)
        buf = torch.empty((nblocks, block_size, width + col_pad), dtype=dtype, device=gen_device)
        buf.normal_(generator=g2)
        cache = buf[:, :, :width]
        for h in range(Hkv):
            cache[:, :, offsets[h] + ranks[h]:offsets[h] + widths[h]] = 0
        k_codes = v_codes = None
    wl = Workload(query=q, kv_cache=cache, block_table=bt, seq_lens=torch.tensor(lengths, dtype=torch.int32),
                  max_seq_len=int(max_seq_len), k_up=k_up, k_ranks=torch.tensor(ranks, dtype=torch.int32),
                  k_head_offsets=torch.tensor(offsets, dtype=torch.int32), k_width=W, v_up_by_q=v_up_by_q,
                  cos_sin_cache=cs, scale=1.0 / math.sqrt(HEAD_DIM), ranks=list(ranks), v_rank=v_rank,
                  lengths=list(lengths), k_codes=k_codes, v_codes=v_codes)
    return wl


def make_quant(lengths, num_heads=32, ranks=None, v_rank=64, seed=0, dtype=torch.bfloat16, max_seq_len=None,
               col_pad=0, device="cuda", peaked=1.0, rotate=True, rank_choices=RANK_CHOICES,
               gen_device="cpu", block_size=BLOCK_SIZE) -> Workload:
    """3.2-bit workload: codes drawn (on `gen_device`), rotated, packed on `device` with pack_kv."""
    from starkv_serve.kernels.paged_quant import HADAMARD_SEED, QuantRow, block_hadamard, k_tables, n_outlier, pack_kv
    gen = torch.Generator(device="cpu").manual_seed(seed)
    H = num_heads
    if ranks is None:
        ranks = [rank_choices[i] for i in torch.randint(0, len(rank_choices), (H,), generator=gen).tolist()]
    widths = [align16(r) for r in ranks]
    offsets = [sum(widths[:h]) for h in range(H)]
    W = sum(widths)
    n = len(lengths)
    max_seq_len = max_seq_len or max(max(lengths), 1)
    bt, nblocks = _page_layout(lengths, gen, block_size=block_size)
    row = QuantRow(W, H, v_rank)

    q = (torch.randn(n, H, HEAD_DIM, generator=gen) * peaked).to(dtype)
    k_up = torch.zeros(W, HEAD_DIM, dtype=torch.float64)
    for h in range(H):
        k_up[offsets[h]:offsets[h] + ranks[h]] = (torch.randn(ranks[h], HEAD_DIM, generator=gen)
                                                  / math.sqrt(ranks[h])).double()
    v_up = (torch.randn(H, v_rank, HEAD_DIM, generator=gen) / math.sqrt(v_rank)).double()
    T = int(sum(lengths))
    if gen_device == "cpu":
        k_codes = torch.randn(T, W, generator=gen)
        v_codes = torch.randn(T, v_rank, generator=gen)
    else:  # benchmark-sized caches: draw on the GPU
        g2 = torch.Generator(device=gen_device).manual_seed(seed + 7919)
        k_codes = torch.randn(T, W, generator=g2, device=gen_device)
        v_codes = torch.randn(T, v_rank, generator=g2, device=gen_device)
    for h in range(H):
        k_codes[:, offsets[h] + ranks[h]:offsets[h] + widths[h]] = 0
    if rotate:
        gk = torch.Generator().manual_seed(HADAMARD_SEED)
        for h in range(H):
            o, r = offsets[h], ranks[h]
            Th = block_hadamard(r, n_outlier(r), gk)
            k_codes[:, o:o + r] = k_codes[:, o:o + r] @ Th.float().to(k_codes.device)
            k_up[o:o + r] = Th.T @ k_up[o:o + r]
        Tv = block_hadamard(v_rank, n_outlier(v_rank), torch.Generator().manual_seed(HADAMARD_SEED))
        v_codes = v_codes @ Tv.float().to(v_codes.device)
        v_up = torch.einsum("rs,hsd->hrd", Tv.T, v_up)
    k_codes = k_codes.to(dtype)
    v_codes = v_codes.to(dtype)
    k_up = k_up.to(dtype)
    v_up_by_q = v_up.to(dtype)
    cs = cos_sin_table(max(max_seq_len, max(lengths) + 1), dtype)

    blk, slot = _token_slots(lengths, bt, block_size)
    slots = (blk * block_size + slot).to(torch.int64)
    buf = torch.randint(0, 256, (nblocks, block_size, row.nbytes + col_pad), generator=gen, dtype=torch.uint8)
    cache = buf[:, :, :row.nbytes]
    nouts, hol, tiles = k_tables(ranks, "cpu")
    wl = Workload(query=q, kv_cache=cache, block_table=bt, seq_lens=torch.tensor(lengths, dtype=torch.int32),
                  max_seq_len=int(max_seq_len), k_up=k_up, k_ranks=torch.tensor(ranks, dtype=torch.int32),
                  k_head_offsets=torch.tensor(offsets, dtype=torch.int32), k_width=W, v_up_by_q=v_up_by_q,
                  cos_sin_cache=cs, scale=1.0 / math.sqrt(HEAD_DIM), ranks=list(ranks), v_rank=v_rank,
                  lengths=list(lengths), quant=True, row=row, k_nouts=nouts, head_of_lane=hol, k_tiles=tiles,
                  k_codes=k_codes, v_codes=v_codes, extra={"slots": slots})
    if device != "cpu":
        wl = wl.to(device)
        pack_kv(wl.k_codes, wl.v_codes, wl.kv_cache, wl.extra["slots"].to(device), row, wl.k_ranks,
                wl.k_head_offsets, wl.k_nouts)
    return wl


def ragged_lengths(seed: int, n: int = 64, lo: int = 1024, hi: int = 8192) -> list:
    """n request lengths drawn uniformly from [lo, hi] with a CPU generator seeded `seed`."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, (n,), generator=g).tolist()
