"""fxlm.prepare_bytes: text files, directories or globs -> byte-level token files.

    python radeon-igpu-forge_amd/fxlm/prepare_bytes.py --out data/demo notes/*.md src/

Front end of ml/fxlm/prepare_bytes.py:19-99 with the same arguments and outputs:
``<out>_train.bin`` / ``<out>_val.bin`` (uint16, one token per byte value) and
``<out>.json`` {vocab_size: 256, tokenizer: "bytes", n_train, n_val, n_files}, written by
``fxlm.train.write_byte_tokens``.  Directories are walked for the ``--ext`` suffixes;
files whose first 8 KB hold a NUL byte are skipped as binary; ``--max-bytes`` truncates
the concatenation.  Needs numpy and the standard library only (no GPU, no torch).
"""
import argparse
import glob
import os
import sys


def build_parser():
    ap = argparse.ArgumentParser(description="text -> byte-level token .bin files")
    ap.add_argument("inputs", nargs="+", help="text files, directories or globs")
    ap.add_argument("--out", required=True, help="output prefix: <out>_train.bin, <out>_val.bin, <out>.json")
    ap.add_argument("--val-frac", type=float, default=0.01)
    ap.add_argument("--max-bytes", type=int, default=0, help="0: no limit; otherwise truncate the input")
    ap.add_argument("--ext", default=".txt,.md,.py",
                    help="comma-separated suffixes taken when walking directories (explicit files "
                         "and globs are taken as given)")
    return ap


def collect_files(inputs, exts):
    """Files named by `inputs`: directories walked for `exts` (lower-case suffixes), globs
    expanded in sorted order, plain names kept; only existing regular files remain."""
    files = []
    for pat in inputs:
        if os.path.isdir(pat):
            for root, _dirs, names in os.walk(pat):
                for n in sorted(names):
                    if n.lower().endswith(exts):
                        files.append(os.path.join(root, n))
        else:
            hits = sorted(glob.glob(pat))
            files += hits if hits else [pat]
    return [f for f in files if os.path.isfile(f)]


def text_files(files):
    """(kept, skipped): files whose first 8 KB contain no NUL byte, and the count of the
    others (binary or unreadable)."""
    kept, skipped = [], 0
    for f in files:
        try:
            with open(f, "rb") as fh:
                head = fh.read(8192)
        except OSError:
            skipped += 1
            continue
        if b"\x00" in head:
            skipped += 1
        else:
            kept.append(f)
    return kept, skipped


def read_bytes(files, max_bytes=0):
    """The files' bytes concatenated in order, cut at max_bytes (0: all of them)."""
    chunks, total = [], 0
    for f in files:
        try:
            with open(f, "rb") as fh:
                data = fh.read()
        except OSError:
            continue
        if max_bytes and total + len(data) > max_bytes:
            data = data[:max_bytes - total]
        chunks.append(data)
        total += len(data)
        if max_bytes and total >= max_bytes:
            break
    return b"".join(chunks)


def main(argv=None):
    args = build_parser().parse_args(argv)
    from fxlm.train import write_byte_tokens

    exts = tuple(e.strip().lower() for e in args.ext.split(",") if e.strip())
    files = collect_files(args.inputs, exts)
    if not files:
        raise SystemExit("no input files: " + " ".join(args.inputs))
    files, skipped = text_files(files)
    if skipped:
        print(f"skipped {skipped} binary or unreadable files")
    if not files:
        raise SystemExit("no text files left after the binary filter")
    print(f"reading {len(files)} files...")
    raw = read_bytes(files, args.max_bytes)
    meta = write_byte_tokens(raw, args.out, val_frac=args.val_frac, n_files=len(files))
    print(f"wrote {args.out}_train.bin ({meta['n_train']:,} tokens) | {args.out}_val.bin "
          f"({meta['n_val']:,}) | {args.out}.json")
    return meta


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    main()
