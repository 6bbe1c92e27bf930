class TensorLayout:
    """Layout of the last three dims of a paged cache page
    (reference quest/utils/utils.py): NHD = [2][S][H][D], HND = [2][H][S][D]."""
    NHD = 0
    HND = 1

    FORMAT2STR = {0: "NHD", 1: "HND"}
