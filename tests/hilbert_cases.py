"""Known answers for the Hilbert order (``pallas_attn.py:41-82``) that follow from the mathematics
of Skilling's transpose algorithm and the reference's lat/lon -> xyz convention, not from running
an implementation. Shared by the oracle tests and the native-library tests.

Top level of the curve. In Skilling's AxestoTranspose ("Programming the Hilbert curve", AIP Conf.
Proc. 707, 2004) the "inverse undo" loop runs from Q = 2**(b-1) down to 2 and only touches the
bits below Q, and so does the final flip; the top bits of the transposed index are therefore the
Gray-encode prefix XOR of the coordinates' top bits, (b0, b0^b1, b0^b1^b2), and the index's three
leading bits are that triple with axis 0 first. Ordering by the index thus visits the eight
octants in reflected Gray-code order of (b0, b1, b2):
000, 001, 011, 010, 110, 111, 101, 100.
With x = cos(lat) cos(lon), y = cos(lat) sin(lon), z = sin(lat) (``pallas_attn.py:76``) and
b = 1 for a positive coordinate, the octant centres (lat +-35.26, lon +-45 / +-135) come out in
the sign order (x, y, z): ---, --+, -++, -+-, ++-, +++, +-+, +--. Any other assignment of the
axes, or a wrong sign convention, reorders them.

Quantisation. A coordinate of -1 maps to 0 and +1 to 2**bits - 1; 0 maps to (2**bits - 1) / 2,
which is a half and rounds to even: 512 at 10 bits, whose top bit is set. So the six axis points
+-x, +-y, +-z land in octants -x: -++, -z: ++-, +x, +y, +z: +++, -y: +-+, i.e. in Gray positions
2, 4, 5, 5, 5, 6.
"""
import numpy as np

GRAY = [0b000, 0b001, 0b011, 0b010, 0b110, 0b111, 0b101, 0b100]  # b0 (x) is the leading bit
_LAT_C = float(np.degrees(np.arcsin(1.0 / np.sqrt(3.0))))         # 35.264 degrees


def octant_centre(octant):
  """(lat, lon) of the centre of the octant with sign bits (x, y, z) = octant (1 = positive)."""
  sx, sy, sz = (octant >> 2) & 1, (octant >> 1) & 1, octant & 1
  lat = _LAT_C if sz else -_LAT_C
  lon = {(1, 1): 45.0, (0, 1): 135.0, (0, 0): -135.0, (1, 0): -45.0}[(sx, sy)]
  return lat, lon


def octant_case(seed=0):
  """Octant centres in a shuffled order: (lat, lon, expected permutation)."""
  rng = np.random.default_rng(seed)
  octs = np.array(GRAY)[rng.permutation(8)]
  lat, lon = np.array([octant_centre(o) for o in octs]).T
  pos = {o: i for i, o in enumerate(octs.tolist())}
  return lat, lon, np.array([pos[o] for o in GRAY])


# +x, -x, +y, -y, +z, -z as (lat, lon).
AXIS_POINTS = {"+x": (0.0, 0.0), "-x": (0.0, 180.0), "+y": (0.0, 90.0), "-y": (0.0, -90.0),
               "+z": (90.0, 0.0), "-z": (-90.0, 0.0)}
# Quantised cells at 10 bits.
AXIS_CELLS = {"+x": (1023, 512, 512), "-x": (0, 512, 512), "+y": (512, 1023, 512), "-y": (512, 0, 512),
              "+z": (512, 512, 1023), "-z": (512, 512, 0)}


def axis_order_ok(perm, names):
  """Whether permutation `perm` of the points `names` visits -x, -z, the three of +++ (any order),
  then -y."""
  got = [names[i] for i in perm]
  return got[0] == "-x" and got[1] == "-z" and set(got[2:5]) == {"+x", "+y", "+z"} and got[5] == "-y"


def skilling_transpose_to_axes(h, bits, dims=3):
  """Coordinates int64[n, dims] of Hilbert indices h (Skilling's TransposetoAxes, the inverse
  routine of the paper, written from its published steps): de-interleave the index into the
  transpose (axis 0 takes the leading bit of each triple), Gray decode, then undo the excess work
  from Q = 2 upwards."""
  h = np.asarray(h, np.int64)
  x = [np.zeros_like(h) for _ in range(dims)]
  for b in range(bits):
    for i in range(dims):
      x[i] |= ((h >> (dims * b + dims - 1 - i)) & 1) << b
  t = x[dims - 1] >> 1
  for i in range(dims - 1, 0, -1):
    x[i] ^= x[i - 1]
  x[0] ^= t
  q = 2
  while q != (1 << bits):
    p = q - 1
    for i in range(dims - 1, -1, -1):
      hi = (x[i] & q) != 0
      x[0] = np.where(hi, x[0] ^ p, x[0])
      swap = np.where(hi, 0, (x[0] ^ x[i]) & p)
      x[0] ^= swap
      x[i] ^= swap
    q <<= 1
  return np.stack(x, -1)
